"""Attention dropout on the GPU: the keep decisions of ``atx_dropout_mask``,
``atx_attn_fwd`` and ``atx_attn_bwd`` against the oracle's restatement
(``oracle/dropout.py``), bit-exact; outputs and gradients against the float64
oracle run with that mask made explicit (``drop = keep / (1 - p)``), to the
contract's tolerances (fp32 1e-5 normwise relative, 16-bit 2e-2 max-abs;
gradients as in ``test_gpu_attention_bwd``).

The reference's dropout is ``F.dropout`` on the softmax weights
(stratego/networks/attention.py:312-313), drawn from torch's Philox stream,
which no other generator reproduces; parity here is "the reference's math
with the same mask", and the mask's statistics are pinned on the CPU
(``tests/test_oracle_dropout.py``).
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from ataraxos_amd import MultiHeadAttention, ops
from oracle.attention import attention as oracle_attention
from oracle.attention import attention_backward as oracle_backward
from oracle.dropout import drop_hash, drop_key, keep_mask
from tests._cases import assert_close, randn, to_np64
from tests.test_gpu_attention_bwd import assert_grad_close

pytestmark = pytest.mark.gpu


def _announce(msg: str) -> None:
    print(f"\n[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("shape,p,seed,offset", [
    ((2, 6, 101, 101), 0.1, 1, 0),
    ((3, 8, 17, 33), 0.5, (1 << 63) + 5, 7),   # 13464 elements: a partial last run of 16
    ((1, 1, 1, 1), 0.3, 9, 9),
    ((4, 2, 64, 64), 0.0, 4, 0),               # p = 0 keeps everything
])
def test_mask_matches_oracle(cuda, shape, p, seed, offset):
    _announce(f"dropout_mask {shape} p={p}")
    got = ops.dropout_mask(*shape, p, seed, offset, device=cuda).cpu().numpy()
    want = keep_mask(*shape, p, seed, offset)
    assert got.dtype == np.uint8 and np.array_equal(got.astype(bool), want)


def test_mask_past_two_to_the_32(cuda):
    """Flat indices past 2^32 use the index's upper word: 4.6e9 decisions,
    checked around the 2^32 boundary and at the end."""
    shape, p, seed, offset = (1100, 8, 512, 1024), 0.25, 77, 3
    _announce(f"dropout_mask {shape} (4.6 GB)")
    keep = ops.dropout_mask(*shape, p, seed, offset, device=cuda).view(-1)
    k0, k1, thresh, _ = drop_key(p, seed, offset)
    n = keep.numel()
    for lo in (0, (1 << 32) - 4096, n - 8192):
        idx = np.arange(lo, lo + 8192, dtype=np.uint64)
        want = drop_hash(idx, k0, k1) >= np.uint32(thresh)
        assert np.array_equal(keep[lo:lo + 8192].cpu().numpy().astype(bool), want), lo
    del keep
    torch.cuda.empty_cache()


def _inputs(b, sq, skv, h, hkv, d, dtype, seed):
    q = randn((b, sq, h, d), seed, dtype)
    k = randn((b, skv, hkv, d), seed + 1, dtype)
    v = randn((b, skv, hkv, d), seed + 2, dtype)
    return q, k, v


def _pad(b, skv, seed):
    g = torch.Generator().manual_seed(seed)
    pad = torch.rand(b, skv, generator=g) < 0.25
    pad[:, 0] = False
    return pad


FWD_CASES = [
    # b, sq, skv, h, hkv, d, causal, padded
    (3, 101, 101, 6, 6, 64, False, False),
    (3, 101, 101, 6, 6, 64, True, False),
    (3, 101, 101, 8, 8, 48, False, True),
    (2, 37, 101, 8, 2, 64, False, False),   # cross-attention shape, GQA
    (2, 300, 64, 4, 4, 48, True, False),
    (5, 1, 17, 4, 4, 64, False, False),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("case", FWD_CASES, ids=lambda c: "x".join(map(str, c[:6])) + ("-c" if c[6] else "") + ("-p" if c[7] else ""))
def test_forward_matches_oracle_with_the_mask(cuda, dtype, case):
    b, sq, skv, h, hkv, d, causal, padded = case
    p, seed, offset = 0.2, 1234 + sq, 5
    _announce(f"fwd dropout {case} {dtype}")
    q, k, v = _inputs(b, sq, skv, h, hkv, d, dtype, seed=sq + d)
    pad = _pad(b, skv, seed) if padded else None
    out = ops.attention_forward(q.to(cuda), k.to(cuda), v.to(cuda), causal=causal,
                                key_padding_mask=None if pad is None else pad.to(cuda),
                                dropout_p=p, dropout_seed=seed, dropout_offset=offset)
    mult = keep_mask(b, h, sq, skv, p, seed, offset) / np.float64(np.float32(1) - np.float32(p))
    want = oracle_attention(to_np64(q), to_np64(k), to_np64(v), causal=causal,
                            key_pad=None if pad is None else pad.numpy(), drop=mult)
    assert_close(out, want, dtype, f"fwd dropout {case}")
    # the same call again gives the same bits; another offset does not
    again = ops.attention_forward(q.to(cuda), k.to(cuda), v.to(cuda), causal=causal,
                                  key_padding_mask=None if pad is None else pad.to(cuda),
                                  dropout_p=p, dropout_seed=seed, dropout_offset=offset)
    assert torch.equal(out, again)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_forward_dropped_weights_are_exactly_the_mask(cuda, dtype):
    """With V = I (S_kv = head_dim = 64) the output row is the dropped
    softmax row itself: its zeros are exactly the dropped weights."""
    b, s, h, d, p, seed = 4, 64, 6, 64, 0.3, 99
    q = randn((b, s, h, d), 5, dtype)
    k = randn((b, s, h, d), 6, dtype)
    v = torch.eye(d, dtype=dtype)[None, :, None, :].expand(b, s, h, d).contiguous()
    out = ops.attention_forward(q.to(cuda), k.to(cuda), v.to(cuda), dropout_p=p, dropout_seed=seed)
    keep = keep_mask(b, h, s, s, p, seed, 0)                      # [b, h, i, j]
    got_zero = (out.float().cpu().numpy() == 0).transpose(0, 2, 1, 3)  # [b, h, i, j]
    assert np.array_equal(got_zero, ~keep)
    # kept weights are P / (1 - p): each row sums to (kept mass) / (1 - p)
    mult = keep / np.float64(np.float32(1) - np.float32(p))
    want = oracle_attention(to_np64(q), to_np64(k), to_np64(v), drop=mult)
    assert_close(out, want, dtype, "V = I")


@pytest.mark.gpu
def test_forward_past_two_to_the_32(cuda):
    """The Move-network layer (6 x 64, S = 101) at a batch whose dropout
    indices pass 2^32 (72000 samples: 4.4e9 weights); sampled samples at the
    start, across the boundary and at the end against the oracle."""
    b, s, h, d, p, seed, offset = 72000, 101, 6, 64, 0.1, 31, 2
    _announce(f"fwd dropout B={b} (indices past 2^32)")
    g = torch.Generator(device=cuda).manual_seed(0)
    q = torch.randn((b, s, h, d), generator=g, device=cuda, dtype=torch.bfloat16)
    k = torch.randn((b, s, h, d), generator=g, device=cuda, dtype=torch.bfloat16)
    v = torch.randn((b, s, h, d), generator=g, device=cuda, dtype=torch.bfloat16)
    out = ops.attention_forward(q, k, v, dropout_p=p, dropout_seed=seed, dropout_offset=offset)
    per_sample = h * s * s
    boundary = (1 << 32) // per_sample
    k0, k1, thresh, _ = drop_key(p, seed, offset)
    scale = np.float64(np.float32(1) / (np.float32(1) - np.float32(p)))
    for bi in (0, boundary - 1, boundary, boundary + 1, b - 1):
        idx = np.arange(bi * per_sample, (bi + 1) * per_sample, dtype=np.uint64).reshape(1, h, s, s)
        mult = (drop_hash(idx, k0, k1) >= np.uint32(thresh)) * scale
        want = oracle_attention(to_np64(q[bi:bi + 1]), to_np64(k[bi:bi + 1]), to_np64(v[bi:bi + 1]), drop=mult)
        assert_close(out[bi:bi + 1], want, torch.bfloat16, f"sample {bi}")
    del q, k, v, out
    torch.cuda.empty_cache()


BWD_CASES = [
    (2, 101, 101, 6, 6, 64, False, False),
    (2, 101, 101, 6, 6, 64, True, False),
    (2, 101, 101, 8, 8, 48, False, True),
    (2, 64, 101, 8, 2, 64, False, False),   # GQA
    (1, 300, 64, 2, 2, 48, True, False),    # two query blocks
    (3, 17, 9, 4, 4, 64, False, False),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("case", BWD_CASES, ids=lambda c: "x".join(map(str, c[:6])) + ("-c" if c[6] else "") + ("-p" if c[7] else ""))
def test_backward_matches_oracle_with_the_mask(cuda, dtype, case):
    b, sq, skv, h, hkv, d, causal, padded = case
    p, seed, offset = 0.15, 4321 + skv, 1
    _announce(f"bwd dropout {case} {dtype}")
    q, k, v = _inputs(b, sq, skv, h, hkv, d, dtype, seed=7 * sq + d)
    go = randn((b, sq, h, d), 3, dtype)
    pad = _pad(b, skv, seed) if padded else None
    dev = [t.to(cuda) for t in (q, k, v, go)]
    kpm = None if pad is None else pad.to(cuda)
    out = ops.attention_forward(dev[0], dev[1], dev[2], causal=causal, key_padding_mask=kpm,
                                dropout_p=p, dropout_seed=seed, dropout_offset=offset)
    dq, dk, dv = ops.attention_backward(dev[0], dev[1], dev[2], out, dev[3], causal=causal, key_padding_mask=kpm,
                                        dropout_p=p, dropout_seed=seed, dropout_offset=offset)
    mult = keep_mask(b, h, sq, skv, p, seed, offset) / np.float64(np.float32(1) - np.float32(p))
    want = oracle_backward(to_np64(q), to_np64(k), to_np64(v), to_np64(go), causal=causal,
                           key_pad=None if pad is None else pad.numpy(), drop=mult)
    for name, got, ref in zip(("dq", "dk", "dv"), (dq, dk, dv), want):
        assert_grad_close(got, ref, f"{name} {case} {dtype}")


def test_autograd_function_replays_the_mask(cuda):
    """ops.attention with autograd: the backward uses the forward's seed."""
    torch.manual_seed(11)
    b, s, h, d, p = 2, 101, 6, 64, 0.1
    q, k, v = (t.to(cuda).requires_grad_(True) for t in _inputs(b, s, s, h, h, d, torch.float32, 21))
    go = randn((b, s, h, d), 22, torch.float32)
    torch.manual_seed(5)
    seed = ops.new_dropout_seed()
    torch.manual_seed(5)
    out = ops.attention(q, k, v, dropout_p=p)
    out.backward(go.to(cuda))
    mult = keep_mask(b, h, s, s, p, seed, 0) / np.float64(np.float32(1) - np.float32(p))
    want_o = oracle_attention(to_np64(q), to_np64(k), to_np64(v), drop=mult)
    assert_close(out, want_o, torch.float32, "autograd fwd")
    want = oracle_backward(to_np64(q), to_np64(k), to_np64(v), to_np64(go), drop=mult)
    for name, t, ref in zip(("dq", "dk", "dv"), (q, k, v), want):
        assert_grad_close(t.grad, ref, f"autograd {name}")


def test_module_trains_with_kernel_dropout(cuda):
    """MultiHeadAttention(384, 6, dropout=0.1) in training runs the HIP
    kernels with dropout: same torch seed, same output; another seed,
    another mask; forward and gradients equal the reference math with the
    kernel's mask applied explicitly (fp32)."""
    torch.manual_seed(0)
    m = MultiHeadAttention(384, 6, dropout=0.1).to(cuda).train()
    assert m.backend == "hip"
    x = randn((2, 101, 384), 8, torch.float32).to(cuda).requires_grad_(True)
    torch.manual_seed(42)
    seed = ops.new_dropout_seed()
    torch.manual_seed(42)
    y = m(x)
    torch.manual_seed(42)
    assert torch.equal(y, m(x))
    torch.manual_seed(43)
    assert not torch.equal(y, m(x))
    # the same layer through torch ops with the mask made explicit
    keep = ops.dropout_mask(2, 6, 101, 101, 0.1, seed, device=cuda).float()
    xr = x.detach().clone().requires_grad_(True)
    q = m.q_proj(xr).view(2, 101, 6, 64).transpose(1, 2)
    k = m.k_proj(xr).view(2, 101, 6, 64).transpose(1, 2)
    v = m.v_proj(xr).view(2, 101, 6, 64).transpose(1, 2)
    probs = torch.softmax(torch.matmul(q, k.transpose(-2, -1).contiguous()) / 8.0, dim=-1)
    probs = probs * keep / (1.0 - torch.tensor(0.1, dtype=torch.float32).item())
    yr = m.out_proj(torch.matmul(probs, v).transpose(1, 2).reshape(2, 101, 384))
    err = (y - yr).abs().max().item() / yr.abs().max().item()
    assert err <= 1e-5, err
    g = randn((2, 101, 384), 9, torch.float32).to(cuda)
    torch.manual_seed(42)
    x.grad = None
    m.zero_grad()
    m(x).backward(g)
    gx, gw = x.grad.clone(), m.q_proj.weight.grad.clone()
    m.zero_grad()
    yr.backward(g)
    for name, got, ref in (("x", gx, xr.grad), ("q_proj.weight", gw, m.q_proj.weight.grad)):
        rel = (got - ref).abs().max().item() / ref.abs().max().item()
        assert rel <= 1e-4, (name, rel)
