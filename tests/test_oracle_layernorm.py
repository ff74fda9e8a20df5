"""The oracle's LayerNorm and pre-LN attention half, pinned on the CPU:
LayerNorm against torch.nn.functional.layer_norm in float64 (the library
routine the reference's nn.LayerNorm calls) and its closed forms (zero mean,
unit biased variance per row before the affine map; a constant row maps to
the bias); the block half against an explicit composition of torch's float64
LayerNorm and nn.MultiheadAttention-free math (the module oracle, itself
pinned in test_oracle_*), plus a planted mistake that must be caught."""

from __future__ import annotations

import numpy as np
import torch

from oracle.attention import layer_norm, mha_forward, preln_attention_half


def test_layer_norm_matches_torch_float64():
    rng = np.random.default_rng(3)
    x = rng.normal(size=(5, 7, 384)) * 3 + 1
    w, b = rng.normal(size=384), rng.normal(size=384)
    for eps in (1e-5, 1e-3):
        ref = torch.nn.functional.layer_norm(torch.from_numpy(x), (384,), torch.from_numpy(w), torch.from_numpy(b), eps)
        np.testing.assert_allclose(layer_norm(x, w, b, eps), ref.numpy(), rtol=0, atol=1e-12)


def test_layer_norm_closed_forms():
    rng = np.random.default_rng(4)
    x = rng.normal(size=(3, 10, 64)) * 5 - 2
    y = layer_norm(x, None, None, 0.0)
    np.testing.assert_allclose(y.mean(axis=-1), 0, atol=1e-12)
    np.testing.assert_allclose((y**2).mean(axis=-1), 1, atol=1e-12)
    b = rng.normal(size=64)
    const = np.full((2, 64), 7.5)
    np.testing.assert_allclose(layer_norm(const, rng.normal(size=64), b, 1e-5), np.broadcast_to(b, (2, 64)), atol=1e-12)


def test_preln_half_composition_and_planted_mistake():
    rng = np.random.default_rng(5)
    e, h = 96, 3
    x = rng.normal(size=(2, 9, e))
    wts = {f"attn.{n}.weight": rng.normal(size=(e, e)) * 0.1 for n in ("q_proj", "k_proj", "v_proj", "out_proj")}
    wts["ln1.weight"], wts["ln1.bias"] = rng.normal(size=e), rng.normal(size=e)
    lnx = torch.nn.functional.layer_norm(torch.from_numpy(x), (e,), torch.from_numpy(wts["ln1.weight"]),
                                         torch.from_numpy(wts["ln1.bias"]), 1e-5).numpy()
    attn_w = {k[5:]: v for k, v in wts.items() if k.startswith("attn.")}
    ref = x + mha_forward(lnx, None, attn_w, h)
    got = preln_attention_half(x, wts, h)
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-12)
    # planted mistake: the residual taken from the normalised rows instead of x
    wrong = lnx + mha_forward(lnx, None, attn_w, h)
    assert np.abs(wrong - got).max() > 1e-2
