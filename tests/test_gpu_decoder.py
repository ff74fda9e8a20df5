"""The Belief decoder stack and the Setup network's token-by-token decode on
the GPU through the HIP kernels, against torch / the CPU math path."""

from __future__ import annotations

import copy
import sys

import pytest
import torch

from ataraxos_amd import SetupDecoder, use_hip_attention
from tests._netlike import SetupLike, belief_decoder

pytestmark = pytest.mark.gpu


def _announce(msg: str) -> None:
    print(f"\n[case] {msg}", flush=True)
    sys.stdout.flush()


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    return ((a.float() - b.float()).abs().max() / b.float().abs().max()).item()


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 3e-2)])
def test_belief_decoder_matches_torch(cuda, dtype, tol):
    """belief_net.py:159-177: causal tgt_mask, memory_key_padding_mask = ~hidden_mask."""
    _announce(f"belief decoder {dtype}")
    torch.manual_seed(0)
    dec = belief_decoder().eval()
    ref = copy.deepcopy(dec).to(cuda, dtype)
    dec = use_hip_attention(dec).to(cuda, dtype)
    b, s = 16, 40
    tgt = torch.randn(b, s, 512, device=cuda, dtype=dtype)
    mem = torch.randn(b, 100, 512, device=cuda, dtype=dtype)
    hidden = torch.rand(b, 100, device=cuda) < 0.4
    hidden[:, 0] = True
    mask = torch.triu(torch.full((s, s), float("-inf"), device=cuda, dtype=dtype), 1)
    with torch.no_grad():
        got = dec(tgt, mem, tgt_mask=mask, memory_key_padding_mask=~hidden)
        want = ref.float()(tgt.float(), mem.float(), tgt_mask=mask.float(), memory_key_padding_mask=~hidden)
    assert torch.isfinite(got).all()
    assert _rel(got, want) <= tol


def test_kernel_mha_refuses_what_it_does_not_cover(cuda):
    m = use_hip_attention(torch.nn.MultiheadAttention(64, 4, batch_first=True)).to(cuda).eval()
    x = torch.randn(2, 8, 64, device=cuda)
    with pytest.raises(NotImplementedError, match="need_weights"):
        m(x, x, x)
    with pytest.raises(NotImplementedError, match="attn_mask"):
        m(x, x, x, need_weights=False, attn_mask=torch.zeros(8, 8, device=cuda))
    out, w = m(x, x, x, need_weights=False)
    assert w is None and out.shape == x.shape


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 3e-2)])
def test_setup_decoder_matches_prefix_recompute(cuda, dtype, tol):
    """Step t of the cached decode equals the reference's full recompute over
    tokens 0..t (selfplay.py:139-146,181), computed on the CPU math path."""
    _announce(f"setup decoder {dtype}")
    torch.manual_seed(1)
    net = SetupLike().eval()
    b, steps = 8, 40
    tokens = torch.randint(0, 12, (b, steps))
    with torch.no_grad():
        v_ref, e_ref, p_ref = net(tokens)  # causal: position t of the full pass = prefix 0..t
    gnet = net.to(cuda, dtype)
    dec = SetupDecoder(gnet, b, capacity=steps)
    worst = 0.0
    for t in range(steps):
        v, e, p = dec.step(tokens[:, t].to(cuda))
        worst = max(worst, _rel(p.cpu(), p_ref[:, t]))
        if t == 0:
            assert _rel(v.cpu(), v_ref) <= tol and _rel(e.cpu(), e_ref) <= tol
    assert worst <= tol
