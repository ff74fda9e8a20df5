"""The committed golden fixtures (``tests/golden/*.npz``, written by
``tests/golden/make_golden.py``): the oracle must still reproduce them (CPU),
and the HIP kernels must match them (GPU)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.attention import attention
from oracle.decode import decode_step
from oracle.policy import kq_logits, kq_probs
from tests._cases import LOWP_ABS_TOL
from tests.golden.make_golden import ATTN_CASES, unpack

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def as_torch(a: np.ndarray) -> torch.Tensor:
    """uint16 fixture -> bf16 tensor; float32 -> float32 tensor."""
    if a.dtype == np.uint16:
        return torch.from_numpy(a.astype(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(a)


# --- CPU: the oracle reproduces the fixtures --------------------------------


@pytest.mark.parametrize("name", list(ATTN_CASES))
def test_oracle_reproduces_attention_fixture(name):
    z = load("attention_cases.npz")
    b, sq, skv, h, hkv, d, causal, has_pad = z[f"{name}/meta"]
    pad = z[f"{name}/key_pad"] if has_pad else None
    o = attention(unpack(z[f"{name}/q"]), unpack(z[f"{name}/k"]), unpack(z[f"{name}/v"]), causal=bool(causal), key_pad=pad)
    np.testing.assert_allclose(o, z[f"{name}/o"], rtol=1e-6, atol=1e-6)


def test_oracle_reproduces_policy_and_decode_fixtures():
    z = load("policy_cases.npz")
    q, k = unpack(z["q"]), unpack(z["k"])
    np.testing.assert_allclose(kq_probs(q, k, z["mask"], 1 / 8), z["probs"], rtol=1e-6, atol=1e-12)
    np.testing.assert_allclose(kq_logits(q, k, z["mask"], 1 / 8), z["logits"], rtol=1e-6, atol=1e-6)
    z = load("decode_cases.npz")
    q, kc, vc = unpack(z["q"]), unpack(z["k_cache"]), unpack(z["v_cache"])
    for i, n in enumerate(z["lens"]):
        np.testing.assert_allclose(decode_step(q, kc[:, :, :n], vc[:, :, :n]), z["o"][i], rtol=1e-6, atol=1e-6)


# --- GPU: the kernels match the fixtures -------------------------------------


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(ATTN_CASES))
def test_kernel_matches_attention_fixture(cuda, name):
    from ataraxos_amd import ops

    z = load("attention_cases.npz")
    b, sq, skv, h, hkv, d, causal, has_pad = z[f"{name}/meta"]
    q, k, v = (as_torch(z[f"{name}/{t}"]).to(cuda) for t in "qkv")
    pad = torch.from_numpy(z[f"{name}/key_pad"]).to(cuda) if has_pad else None
    out = ops.attention_forward(q, k, v, causal=bool(causal), key_padding_mask=pad).cpu().double().numpy()
    ref = z[f"{name}/o"].astype(np.float64)
    err = np.abs(out - ref).max()
    if q.dtype == torch.float32:
        assert err <= 1e-5 * np.abs(ref).max()
    else:
        assert err <= LOWP_ABS_TOL


@pytest.mark.gpu
def test_kernels_match_policy_and_decode_fixtures(cuda):
    from ataraxos_amd import ops

    z = load("policy_cases.npz")
    q, k = as_torch(z["q"]).to(cuda), as_torch(z["k"]).to(cuda)
    mask = torch.from_numpy(z["mask"]).to(cuda)
    probs = ops.kq_policy(q, k, mask).cpu().double().numpy()
    assert (probs[~z["mask"].reshape(4, -1)] == 0).all()
    assert np.abs(probs - z["probs"]).max() <= LOWP_ABS_TOL
    assert probs[3, 42 * 100 + 17] == 1.0
    logits = ops.kq_policy(q, k, mask, output="logits").cpu().double().numpy()
    legal = z["mask"].reshape(4, -1)
    assert (logits[~legal] == np.float32(-1e10)).all()
    assert np.abs(logits[legal] - z["logits"][legal]).max() <= LOWP_ABS_TOL
    z = load("decode_cases.npz")
    q, kc, vc = (as_torch(z[t]).to(cuda) for t in ("q", "k_cache", "v_cache"))
    for i, n in enumerate(z["lens"]):
        out = ops.attention_decode(q, kc, vc, int(n)).cpu().double().numpy()
        assert np.abs(out - z["o"][i]).max() <= LOWP_ABS_TOL
