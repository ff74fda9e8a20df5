"""The attention half of the reference's pre-LN block, ``x + attn(ln1(x))``
(stratego/networks/transformer.py:143), as one launch of the persistent
fused layer (LayerNorm on the X rows in LDS, residual added at the Y store),
against the float64 oracle (``oracle.attention.preln_attention_half``).

Tolerance: the contract's 16-bit figure, 2e-2 max-abs, plus half a bf16/fp16
unit in the last place of the reference value: the block's output is a
16-bit sum ``x + y`` whose own final rounding (which any 16-bit
implementation of the block performs, the reference's bf16 modules included)
is up to half an ulp of |x + y|, i.e. 0.0156 for values in [4, 8).
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from ataraxos_amd import PreLNTransformerBlock, ops
from oracle.attention import preln_attention_half
from tests._cases import randn, to_np64

pytestmark = pytest.mark.gpu

NAMES = ("q_proj", "k_proj", "v_proj", "out_proj")


def _announce(msg: str) -> None:
    print(f"\n[case] {msg}", flush=True)
    sys.stdout.flush()


def _half_ulp(ref: np.ndarray, dtype) -> np.ndarray:
    mant = 8 if dtype == torch.bfloat16 else 11  # significand bits incl. the implicit one
    e = np.floor(np.log2(np.maximum(np.abs(ref), 2.0**-14)))
    return 0.5 * 2.0 ** (e - (mant - 1))


def _block_params(e, dtype, seed, bias):
    g = torch.Generator().manual_seed(seed)
    ws = [(torch.randn(e, e, generator=g) * 0.02).to(dtype) for _ in range(4)]
    bs = [(torch.randn(e, generator=g) * 0.02).to(dtype) for _ in range(4)] if bias else [None] * 4
    lw = (1.0 + 0.1 * torch.randn(e, generator=g)).to(dtype)
    lb = (0.1 * torch.randn(e, generator=g)).to(dtype)
    return ws, bs, lw, lb


def _oracle(x, ws, bs, lw, lb, causal, eps):
    wts = {f"attn.{n}.weight": to_np64(w) for n, w in zip(NAMES, ws)}
    wts.update({f"attn.{n}.bias": to_np64(t) for n, t in zip(NAMES, bs) if t is not None})
    wts["ln1.weight"] = to_np64(lw)
    if lb is not None:
        wts["ln1.bias"] = to_np64(lb)
    return preln_attention_half(to_np64(x), wts, 6, causal=causal, eps=eps)


def _check(got, ref, dtype):
    got = to_np64(got)
    assert np.isfinite(got).all()
    err = np.abs(got - ref)
    bound = 2e-2 + _half_ulp(ref, dtype)
    worst = float(np.max(err - bound))
    assert worst <= 0, f"max excess {worst:.3e}, max-abs {float(err.max()):.3e}"


@pytest.mark.parametrize(
    "b,l,dtype,causal,bias,ln_bias,inplace,x_view",
    [
        (4, 100, torch.bfloat16, False, False, True, False, False),
        (3, 101, torch.bfloat16, False, True, True, False, False),
        (5, 65, torch.float16, False, False, False, False, False),
        (300, 97, torch.bfloat16, False, False, True, True, False),
        (4, 80, torch.bfloat16, True, True, True, False, True),
        (513, 100, torch.bfloat16, False, False, True, False, False),
    ],
)
def test_block_half_against_the_oracle(cuda, b, l, dtype, causal, bias, ln_bias, inplace, x_view):
    e = 384
    _announce(f"block half b={b} l={l} {dtype} causal={causal} bias={bias} ln_bias={ln_bias} inplace={inplace} view={x_view}")
    x = randn((b, l, e), 900 + l + b, dtype)
    ws, bs, lw, lb = _block_params(e, dtype, 901 + l, bias)
    lb = lb if ln_bias else None
    eps = 1e-5
    if x_view:
        big = torch.full((b, l + 3, e + 64), float("nan"), dtype=dtype)
        big[:, :l, :e] = x
        xd = big.to(cuda)[:, :l, :e]
    else:
        xd = x.to(cuda)
    kw = dict(num_heads=6, b_q=None, b_k=None, b_v=None, b_o=None, causal=causal, repack=True,
              ln_weight=lw.to(cuda), ln_bias=None if lb is None else lb.to(cuda), ln_eps=eps, residual=True)
    kw.update({k: (t.to(cuda) if t is not None else None) for k, t in zip(("b_q", "b_k", "b_v", "b_o"), bs)})
    wd = [w.to(cuda) for w in ws]
    if inplace:
        y = ops.mha_forward(xd, *wd, out=xd, **kw)
        assert y.data_ptr() == xd.data_ptr()
    else:
        y = ops.mha_forward(xd, *wd, **kw)
    torch.cuda.synchronize()
    rows = list(range(b)) if b <= 8 else [0, 1, b // 2, b - 2, b - 1, 255, 256]
    ref = _oracle(x[rows], ws, bs, lw, lb, causal, eps)
    _check(y[rows], ref, dtype)
    if x_view:
        assert torch.isnan(xd.as_strided((b, 3, e + 64), (xd.stride(0), e + 64, 1), l * (e + 64)).float()).all()


def test_block_half_full_batch_c3(cuda):
    """BASELINE config 3's layer as a pre-LN block half at B=4096, L=100,
    sampled rows against the oracle on those rows alone."""
    b, l, e = 4096, 100, 384
    _announce(f"block half full batch b={b}")
    x = randn((b, l, e), 950, torch.bfloat16)
    ws, _, lw, lb = _block_params(e, torch.bfloat16, 951, False)
    y = ops.mha_forward(x.to(cuda), *[w.to(cuda) for w in ws], num_heads=6, repack=True,
                        ln_weight=lw.to(cuda), ln_bias=lb.to(cuda), residual=True)
    torch.cuda.synchronize()
    rows = [0, 1, 255, 256, 2047, 4095] + list(range(91, 4000, 577))
    _check(y[rows], _oracle(x[rows], ws, [None] * 4, lw, lb, False, 1e-5), torch.bfloat16)


def test_block_half_eight_layer_chain(cuda):
    """x <- x + MHA_l(LN_l(x)) for 8 layers with N(0, 0.02) weights, each a
    single launch, against the oracle chained in float64 (which never rounds
    between layers: the tolerance grows with the chain, 2e-2 per layer)."""
    b, l, e = 6, 100, 384
    _announce("block half 8-layer chain")
    x0 = randn((b, l, e), 960, torch.bfloat16)
    xd = x0.to(cuda)
    ref = to_np64(x0)
    for layer in range(8):
        ws, _, lw, lb = _block_params(e, torch.bfloat16, 961 + layer, False)
        xd = ops.mha_forward(xd, *[w.to(cuda) for w in ws], num_heads=6, repack=True,
                             ln_weight=lw.to(cuda), ln_bias=lb.to(cuda), residual=True)
        wts = {f"attn.{n}.weight": to_np64(w) for n, w in zip(NAMES, ws)}
        wts["ln1.weight"], wts["ln1.bias"] = to_np64(lw), to_np64(lb)
        ref = preln_attention_half(ref, wts, 6)
    torch.cuda.synchronize()
    got = to_np64(xd)
    err = float(np.max(np.abs(got - ref)))
    assert err <= 8 * 2e-2, err


def test_module_block_takes_the_one_launch_half(cuda, monkeypatch):
    """PreLNTransformerBlock(384, 6, 1536) in inference: the attention half is
    one launch with LayerNorm and residual; the block output equals the
    unfused composition within the 16-bit tolerance (the feed-forward half
    is the same torch code in both)."""
    _announce("PreLNTransformerBlock fused half")
    torch.manual_seed(12)
    blk = PreLNTransformerBlock(384, 6, 1536).to(cuda, torch.bfloat16).eval()
    with torch.no_grad():
        blk.ln1.weight.mul_(1.1)
        blk.ln1.bias.add_(0.05)
    x = randn((5, 100, 384), 970, torch.bfloat16).to(cuda)
    seen = []
    real = ops.mha_forward
    monkeypatch.setattr(ops, "mha_forward", lambda *a, **k: seen.append(k.get("residual")) or real(*a, **k))
    with torch.no_grad():
        fused = blk(x)
        blk.fuse_block = False
        unfused = blk(x)
    torch.cuda.synchronize()
    assert seen and seen[0] is True
    err = (fused.float() - unfused.float()).abs()
    tol = 3e-2 + torch.from_numpy(_half_ulp(unfused.float().cpu().double().numpy(), torch.bfloat16)).to(cuda)
    assert bool((err <= tol).all()), float(err.max())


def test_rejects_unsupported_block_shapes(cuda):
    x = torch.zeros(2, 40, 384, device=cuda, dtype=torch.bfloat16)
    w = torch.zeros(384, 384, device=cuda, dtype=torch.bfloat16)
    lw = torch.ones(384, device=cuda, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError, match="pre-LN"):
        ops.mha_forward(x, w, w, w, w, num_heads=6, ln_weight=lw, residual=True)
    with pytest.raises(ValueError, match="ln_bias"):
        ops.mha_forward(x, w, w, w, w, num_heads=6, ln_bias=lw)
