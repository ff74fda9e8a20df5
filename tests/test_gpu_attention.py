"""Parity of the fused HIP attention kernel against the float64 oracle.

Every case draws seeded inputs on the CPU, runs ``atx_attn_fwd`` through the
C ABI (``ataraxos_amd.ops.attention_forward``) and compares with
``oracle.attention.attention`` under the contract's tolerances
(``tests/_cases.py``).
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from ataraxos_amd import ops
from oracle.attention import attention as oracle_attention
from tests._cases import assert_close, randn, to_np64

pytestmark = pytest.mark.gpu


def _announce(msg: str) -> None:
    print(f"\n[case] {msg}", flush=True)
    sys.stdout.flush()


def _on_gpu(pad, cuda, view):
    """The padding mask on the GPU; with ``view``, as columns 1 .. skv of a
    wider mask whose other columns are True, so that its rows start at odd
    addresses with an odd stride (the kernels' byte-load path)."""
    if not view:
        return pad.to(cuda)
    b, skv = pad.shape
    big = torch.ones(b, skv + 3, dtype=torch.bool)
    big[:, 1 : skv + 1] = pad
    return big.to(cuda)[:, 1 : skv + 1]


def run_case(cuda, b, sq, skv, h, hkv, d, dtype, causal=False, pad_p=None, seed=0, scale=None, pad_view=False):
    _announce(f"b={b} sq={sq} skv={skv} h={h} hkv={hkv} d={d} {dtype} causal={causal} pad={pad_p}")
    q = randn((b, sq, h, d), seed, dtype)
    k = randn((b, skv, hkv, d), seed + 1, dtype)
    v = randn((b, skv, hkv, d), seed + 2, dtype)
    pad = None
    if pad_p is not None:
        g = torch.Generator().manual_seed(seed + 3)
        pad = torch.rand(b, skv, generator=g) < pad_p
    out = ops.attention_forward(
        q.to(cuda), k.to(cuda), v.to(cuda), causal=causal, scale=scale,
        key_padding_mask=None if pad is None else _on_gpu(pad, cuda, pad_view),
    )
    torch.cuda.synchronize()
    ref = oracle_attention(to_np64(q), to_np64(k), to_np64(v), causal=causal, scale=scale,
                           key_pad=None if pad is None else pad.numpy())
    return assert_close(out, ref, dtype, f"attn b={b} sq={sq} skv={skv} d={d} {dtype}")


# --- the BASELINE configurations ------------------------------------------


def test_config1_fp32_move_layer(cuda):
    """C1: fp32, B=64, L=100, 6 heads x 64, no mask, scale 1/8."""
    run_case(cuda, 64, 100, 100, 6, 6, 64, torch.float32, seed=43)


def test_config3_bf16_move_layer_subset(cuda):
    """C3 shape (L=100, 6x64, bf16) at B=256: full oracle comparison."""
    run_case(cuda, 256, 100, 100, 6, 6, 64, torch.bfloat16, seed=45)


def test_config3_bf16_full_batch_properties(cuda):
    """C3 at the full B=4096: 32 sampled batch rows against the oracle, and
    batch-position independence (a sub-batch gives bit-identical rows)."""
    b, l, h, d = 4096, 100, 6, 64
    _announce(f"full C3 b={b}")
    q = randn((b, l, h, d), 45, torch.bfloat16).to(cuda)
    k = randn((b, l, h, d), 46, torch.bfloat16).to(cuda)
    v = randn((b, l, h, d), 47, torch.bfloat16).to(cuda)
    out = ops.attention_forward(q, k, v)
    idx = torch.tensor([0, 1, 2, 3, 511, 1024, 2047, 2048, 3000, 4095] + list(range(100, 4000, 176)))
    ref = oracle_attention(to_np64(q[idx]), to_np64(k[idx]), to_np64(v[idx]))
    assert_close(out[idx.to(cuda)], ref, torch.bfloat16, "C3 sampled rows")
    sub = ops.attention_forward(q[2000:2100], k[2000:2100], v[2000:2100])
    torch.cuda.synchronize()
    assert torch.equal(sub, out[2000:2100])


# --- shape coverage ---------------------------------------------------------

SEQS = [1, 10, 16, 17, 31, 32, 33, 92, 100, 101, 128, 200, 256]


@pytest.mark.parametrize("s", SEQS)
def test_bf16_seq_lengths(cuda, s):
    run_case(cuda, 3, s, s, 4, 4, 64, torch.bfloat16, seed=s)


@pytest.mark.parametrize("d", [16, 32, 48, 64, 80, 96, 112, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_head_dims(cuda, d, dtype):
    run_case(cuda, 2, 101, 101, 3, 3, d, dtype, seed=d)


@pytest.mark.parametrize("s", [1, 17, 100, 256])
def test_fp32_seq_lengths(cuda, s):
    run_case(cuda, 2, s, s, 4, 4, 64, torch.float32, seed=s + 7)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("s", [1, 10, 40, 92, 100, 129])
def test_causal(cuda, dtype, s):
    run_case(cuda, 2, s, s, 8, 8, 64, dtype, causal=True, seed=s + 11)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("sq,skv", [(10, 50), (40, 100), (100, 40), (1, 256), (7, 3)])
def test_cross_attention(cuda, dtype, sq, skv):
    run_case(cuda, 2, sq, skv, 8, 8, 64, dtype, seed=sq * 3 + skv)


@pytest.mark.parametrize("sq,skv", [(10, 30), (40, 40)])
def test_causal_rectangular_top_left(cuda, sq, skv):
    """Causal with S_q != S_kv keeps the reference's top-left alignment."""
    run_case(cuda, 2, sq, skv, 4, 4, 32, torch.float32, causal=True, seed=sq + skv)


@pytest.mark.parametrize("h,hkv", [(8, 2), (8, 4), (8, 1), (6, 3)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gqa(cuda, h, hkv, dtype):
    run_case(cuda, 2, 33, 33, h, hkv, 32, dtype, seed=h * 10 + hkv)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("causal", [False, True])
def test_key_padding(cuda, dtype, causal):
    """Belief-decoder cross-attention shape: 40 queries over 100 keys with a
    key-padding mask (True = ignore)."""
    run_case(cuda, 4, 40, 100, 8, 8, 64, dtype, causal=causal, pad_p=0.6, seed=5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fully_masked_rows_are_nan(cuda, dtype):
    """All keys padded out: NaN, as softmax over an all -inf row gives."""
    b, sq, skv, h, d = 2, 5, 20, 2, 32
    q = randn((b, sq, h, d), 1, dtype)
    k = randn((b, skv, h, d), 2, dtype)
    v = randn((b, skv, h, d), 3, dtype)
    pad = torch.zeros(b, skv, dtype=torch.bool)
    pad[1] = True
    out = ops.attention_forward(q.to(cuda), k.to(cuda), v.to(cuda), key_padding_mask=pad.to(cuda)).cpu()
    assert torch.isnan(out[1]).all()
    assert torch.isfinite(out[0]).all()
    ref = oracle_attention(to_np64(q), to_np64(k), to_np64(v), key_pad=pad.numpy())
    assert_close(out, ref, dtype, "fully masked")


def test_scale_argument(cuda):
    run_case(cuda, 2, 50, 50, 4, 4, 64, torch.bfloat16, seed=9, scale=0.3)


def test_strided_packed_qkv_views(cuda):
    """Q/K/V as strided views of one packed [B, S, 3E] projection output."""
    b, s, h, d = 3, 100, 6, 64
    e = h * d
    packed = randn((b, s, 3 * e), 21, torch.bfloat16)
    q = packed[..., :e].view(b, s, h, d)
    k = packed[..., e : 2 * e].view(b, s, h, d)
    v = packed[..., 2 * e :].view(b, s, h, d)
    pc = packed.to(cuda)
    out = ops.attention_forward(pc[..., :e].view(b, s, h, d), pc[..., e : 2 * e].view(b, s, h, d),
                                pc[..., 2 * e :].view(b, s, h, d))
    ref = oracle_attention(to_np64(q), to_np64(k), to_np64(v))
    assert_close(out, ref, torch.bfloat16, "packed views")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("sq,skv", [(37, 100), (100, 100), (5, 41), (1, 1)])
def test_rows_past_the_sequence_are_neither_read_nor_written(cuda, dtype, sq, skv):
    """Q/K/V/O as the first rows of longer buffers: K/V rows past S_kv and Q
    rows past S_q hold NaN, the output buffer's rows past S_q hold a sentinel.
    The result must match the oracle and the sentinel must survive."""
    _announce(f"guard rows sq={sq} skv={skv} {dtype}")
    b, h, d, extra = 3, 6, 64, 24
    q = randn((b, sq, h, d), 51, dtype)
    k = randn((b, skv, h, d), 52, dtype)
    v = randn((b, skv, h, d), 53, dtype)
    nan = float("nan")
    qb = torch.full((b, sq + extra, h, d), nan, dtype=dtype)
    kb = torch.full((b, skv + extra, h, d), nan, dtype=dtype)
    vb = torch.full((b, skv + extra, h, d), nan, dtype=dtype)
    qb[:, :sq], kb[:, :skv], vb[:, :skv] = q, k, v
    ob = torch.full((b, sq + extra, h, d), 7.0, dtype=dtype, device=cuda)
    qb, kb, vb = qb.to(cuda), kb.to(cuda), vb.to(cuda)
    out = ops.attention_forward(qb[:, :sq], kb[:, :skv], vb[:, :skv], out=ob[:, :sq])
    torch.cuda.synchronize()
    assert (ob[:, sq:] == 7.0).all()
    ref = oracle_attention(to_np64(q), to_np64(k), to_np64(v))
    assert_close(out, ref, dtype, f"guard rows sq={sq} skv={skv}")


def test_single_row_with_arbitrary_sequence_stride(cuda):
    """A length-1 sequence's stride is meaningless (torch may report any
    value); the call must not depend on it."""
    _announce("seq 1 odd strides")
    b, h, d = 4, 6, 64
    base = randn((b, h, 3, d), 61, torch.bfloat16)
    q = base[:, :, 0:1].permute(0, 2, 1, 3)  # [b, 1, h, d], stride_s = d
    k = base[:, :, 1:2].permute(0, 2, 1, 3)
    v = base[:, :, 2:3].permute(0, 2, 1, 3)
    qs, ks, vs = (t.as_strided(t.shape, (t.stride(0), 3, t.stride(2), 1)) for t in (q, k, v))
    bc = base.to(cuda)
    gq, gk, gv = (bc[:, :, i : i + 1].permute(0, 2, 1, 3) for i in range(3))
    gq, gk, gv = (t.as_strided(t.shape, (t.stride(0), 3, t.stride(2), 1), t.storage_offset()) for t in (gq, gk, gv))
    out = ops.attention_forward(gq, gk, gv)
    ref = oracle_attention(to_np64(qs), to_np64(ks), to_np64(vs))
    assert_close(out, ref, torch.bfloat16, "seq 1")


def test_determinism(cuda):
    q = randn((8, 100, 6, 64), 1, torch.bfloat16).to(cuda)
    k = randn((8, 100, 6, 64), 2, torch.bfloat16).to(cuda)
    v = randn((8, 100, 6, 64), 3, torch.bfloat16).to(cuda)
    a = ops.attention_forward(q, k, v)
    b = ops.attention_forward(q, k, v)
    assert torch.equal(a, b)


def test_rejects_unsupported_shapes(cuda):
    q = torch.zeros(1, 4, 2, 8, device=cuda, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="head_dim"):
        ops.attention_forward(q, q, q)
    q = torch.zeros(1, 300, 1, 64, device=cuda, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="seq_kv"):
        ops.attention_forward(q, q, q)


def test_large_logits_are_stable(cuda):
    """Scores of magnitude ~1e3: the max-shifted softmax stays finite."""
    q = randn((2, 64, 2, 64), 5, torch.float32) * 30
    k = randn((2, 64, 2, 64), 6, torch.float32) * 30
    v = randn((2, 64, 2, 64), 7, torch.float32)
    out = ops.attention_forward(q.to(cuda), k.to(cuda), v.to(cuda))
    assert torch.isfinite(out).all()
    ref = oracle_attention(to_np64(q), to_np64(k), to_np64(v))
    np.testing.assert_allclose(to_np64(out), ref, rtol=0, atol=1e-4 * np.abs(ref).max())


@pytest.mark.parametrize("skv,dtype,view", [(129, torch.bfloat16, False), (200, torch.float16, True), (256, torch.bfloat16, False), (256, torch.float32, True)])
def test_key_padding_long_rows(cuda, skv, dtype, view):
    """Key padding over 129..256 keys (every lane of the per-lane padding
    words), with the mask rows 4-byte aligned or at odd addresses."""
    run_case(cuda, 3, 48, skv, 4, 4, 64, dtype, pad_p=0.5, seed=600 + skv, pad_view=view)
