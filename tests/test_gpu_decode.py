"""Parity of the KV-cache decode kernel against the full-recompute oracle."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from ataraxos_amd import KVCache, ops
from oracle.decode import decode_step, full_recompute_last_row
from tests._cases import assert_close, randn, to_np64

pytestmark = pytest.mark.gpu


def _announce(msg: str) -> None:
    print(f"\n[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("d", [8, 16, 32, 48, 64, 128, 256])
def test_decode_matches_oracle(cuda, dtype, d):
    b, h, t, cap = 5, 4, 37, 40
    _announce(f"decode b={b} h={h} t={t} d={d} {dtype}")
    q = randn((b, h, d), d, dtype)
    kc = randn((b, h, cap, d), d + 1, dtype)
    vc = randn((b, h, cap, d), d + 2, dtype)
    out = ops.attention_decode(q.to(cuda), kc.to(cuda), vc.to(cuda), t)
    ref = decode_step(to_np64(q), to_np64(kc)[:, :, :t], to_np64(vc)[:, :, :t])
    assert_close(out, ref, dtype, f"decode d={d}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_config5_incremental_decode(cuda, dtype):
    """C5 scaled to B=64: 4 layers x 40 steps, each step appended through
    k_new/v_new and compared with the last row of the full causal recompute."""
    b, h, d, steps, layers = 64, 8, 64, 40, 4
    _announce(f"C5 incremental b={b} {dtype}")
    qs = randn((layers, b, steps, h, d), 47, dtype)
    ks = randn((layers, b, steps, h, d), 48, dtype)
    vs = randn((layers, b, steps, h, d), 49, dtype)
    cache = KVCache(layers, b, h, steps, d, dtype=dtype, device=cuda)
    qd, kd, vd = qs.to(cuda), ks.to(cuda), vs.to(cuda)
    worst = 0.0
    for t in range(steps):
        for layer in range(layers):
            out = cache.step(layer, qd[layer, :, t], kd[layer, :, t], vd[layer, :, t])
            if t in (0, 1, 7, 20, 39):
                ref = full_recompute_last_row(
                    to_np64(qs[layer, :, : t + 1]), to_np64(ks[layer, :, : t + 1]), to_np64(vs[layer, :, : t + 1])
                )
                worst = max(worst, assert_close(out, ref, dtype, f"step {t} layer {layer}"))
        cache.advance()
    # The cache now holds every appended row.
    torch.cuda.synchronize()
    assert torch.equal(cache.keys(2).cpu(), ks[2].transpose(1, 2).contiguous())
    assert torch.equal(cache.values(3).cpu(), vs[3].transpose(1, 2).contiguous())


def test_config5_full_batch_properties(cuda):
    """C5 at B=8192, t=40: sampled rows against the oracle and batch-position
    independence."""
    b, h, d, t = 8192, 8, 64, 40
    _announce(f"C5 full b={b}")
    q = randn((b, h, d), 1, torch.bfloat16).to(cuda)
    kc = randn((b, h, t, d), 2, torch.bfloat16).to(cuda)
    vc = randn((b, h, t, d), 3, torch.bfloat16).to(cuda)
    out = ops.attention_decode(q, kc, vc, t)
    idx = torch.tensor([0, 1, 4095, 4096, 8191, 1234, 777])
    ref = decode_step(to_np64(q[idx]), to_np64(kc[idx]), to_np64(vc[idx]))
    assert_close(out[idx.to(cuda)], ref, torch.bfloat16, "C5 full sampled")
    sub = ops.attention_decode(q[100:200], kc[100:200], vc[100:200], t)
    torch.cuda.synchronize()
    assert torch.equal(sub, out[100:200])


def test_per_sample_lengths_and_gqa(cuda):
    b, h, hkv, d, cap = 6, 8, 2, 64, 50
    q = randn((b, h, d), 1, torch.float32)
    kc = randn((b, hkv, cap, d), 2, torch.float32)
    vc = randn((b, hkv, cap, d), 3, torch.float32)
    lens = torch.tensor([1, 2, 17, 40, 50, 33], dtype=torch.int32)
    out = ops.attention_decode(q.to(cuda), kc.to(cuda), vc.to(cuda), lens.to(cuda)).cpu()
    for i in range(b):
        n = int(lens[i])
        ref = decode_step(to_np64(q[i : i + 1]), to_np64(kc[i : i + 1, :, :n]), to_np64(vc[i : i + 1, :, :n]))
        assert_close(out[i : i + 1], ref, torch.float32, f"sample {i} len {n}")


def test_zero_length_gives_nan(cuda):
    q = randn((2, 2, 64), 1, torch.float32).to(cuda)
    kc = randn((2, 2, 8, 64), 2, torch.float32).to(cuda)
    lens = torch.tensor([0, 3], dtype=torch.int32, device=cuda)
    out = ops.attention_decode(q, kc, kc, lens).cpu()
    assert torch.isnan(out[0]).all() and torch.isfinite(out[1]).all()


def test_decode_equals_causal_recompute_per_step(cuda):
    """Each step equals row t of the fused causal attention kernel too."""
    b, s, h, d = 3, 40, 8, 64
    q = randn((b, s, h, d), 11, torch.float32).to(cuda)
    k = randn((b, s, h, d), 12, torch.float32).to(cuda)
    v = randn((b, s, h, d), 13, torch.float32).to(cuda)
    full = ops.attention_forward(q, k, v, causal=True)
    kc = k.transpose(1, 2).contiguous()
    vc = v.transpose(1, 2).contiguous()
    for t in (1, 2, 20, 40):
        step = ops.attention_decode(q[:, t - 1], kc, vc, t)
        np.testing.assert_allclose(step.cpu().numpy(), full[:, t - 1].cpu().numpy(), rtol=0, atol=2e-6)


def test_cache_views_wider_than_4gib(cuda):
    """Caches whose batch stride makes one launch's extent exceed 4 GiB: the
    library splits the launch by batch (the kernel uses 32-bit offsets).  The
    views cover 10 batch rows 2^28 elements apart (~4.5 GiB each)."""
    _announce("decode over > 4 GiB cache views, with k_new/v_new")
    b, h, t, d = 10, 2, 8, 64
    sb = 1 << 28
    q = randn((b, h, d), 71, torch.bfloat16)
    kvals = randn((b, h, t, d), 72, torch.bfloat16)
    vvals = randn((b, h, t, d), 73, torch.bfloat16)
    kn = randn((b, h, d), 74, torch.bfloat16)
    vn = randn((b, h, d), 75, torch.bfloat16)
    caches = []
    for vals in (kvals, vvals):
        buf = torch.zeros(sb * (b - 1) + h * t * d, dtype=torch.bfloat16, device=cuda)
        view = buf.as_strided((b, h, t, d), (sb, t * d, d, 1))
        view.copy_(vals.to(cuda))
        caches.append((buf, view))
    (kbuf, kc), (vbuf, vc) = caches
    out = ops.attention_decode(q.to(cuda), kc, vc, t, kn.to(cuda), vn.to(cuda))
    torch.cuda.synchronize()
    kref, vref = to_np64(kvals), to_np64(vvals)
    kref[:, :, t - 1], vref[:, :, t - 1] = to_np64(kn), to_np64(vn)
    assert_close(out, decode_step(to_np64(q), kref, vref), torch.bfloat16, "decode > 4 GiB")
    assert torch.equal(kc[:, :, t - 1].cpu(), kn) and torch.equal(vc[:, :, t - 1].cpu(), vn)
    del kbuf, vbuf, caches
