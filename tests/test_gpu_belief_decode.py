"""Incremental Belief decoding (``BeliefDecoder``) against the network's own
full forward, the computation the reference's ``BeliefSampler`` repeats per
token (stratego/search/belief_sampler.py:84-99).

Criterion (the decode rows' own): the logits of step t equal the last row of
the full decoder over the same t + 1 tokens; the sampler's step-j
probabilities equal the softmax of the full forward's last row over the drawn
tokens followed by the placeholder 0.  fp32: ``max|a - b| <= 1e-4 * max|b|``
(the two paths sum in different orders); bf16: 2e-2 max-abs on probabilities.
"""

from __future__ import annotations

import sys

import pytest
import torch

from ataraxos_amd import BeliefDecoder
from tests._netlike import BeliefLike

pytestmark = pytest.mark.gpu


def _setup(cuda, dtype, seed, b=6):
    torch.manual_seed(seed)
    net = BeliefLike().to(cuda, dtype).eval()
    g = torch.Generator().manual_seed(seed)
    info = torch.randn(b, 32, 10, 10, generator=g).to(cuda, dtype)
    hidden = torch.rand(b, 100, generator=g) < 0.4
    hidden[:, 7] = True
    return net, info, hidden.to(cuda)


def test_step_logits_equal_full_forward_last_row(cuda):
    print("\n[case] belief decode steps fp32", flush=True)
    sys.stdout.flush()
    net, info, hidden = _setup(cuda, torch.float32, 1)
    tokens = torch.randint(0, 12, (info.shape[0], 12), generator=torch.Generator().manual_seed(2)).to(cuda)
    dec = BeliefDecoder(net, info, hidden)
    with torch.no_grad():
        for t in range(tokens.shape[1]):
            got = dec.step(tokens[:, t])
            want = net(info, hidden, tokens[:, : t + 1])[:, -1]
            err = (got - want).abs().max().item()
            assert err <= 1e-4 * want.abs().max().item(), (t, err)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
def test_sampler_probabilities_follow_the_reference_convention(cuda, dtype, tol):
    print(f"\n[case] belief sampler {dtype}", flush=True)
    sys.stdout.flush()
    net, info, hidden = _setup(cuda, dtype, 3)
    dec = BeliefDecoder(net, info, hidden)
    toks, probs = dec.sample(10, generator=torch.Generator(device=cuda).manual_seed(4), return_probs=True)
    assert toks.shape == (info.shape[0], 10) and ((toks >= 0) & (toks < 12)).all()
    with torch.no_grad():
        for j in range(10):
            seq = torch.cat([toks[:, :j], torch.zeros_like(toks[:, :1])], dim=1)
            want = torch.softmax(net(info, hidden, seq)[:, -1].float(), dim=-1)
            err = (probs[:, j] - want).abs().max().item()
            bound = tol * (want.abs().max().item() if dtype == torch.float32 else 1.0)
            assert err <= bound, (j, err)


def test_sampling_is_reproducible_and_resettable(cuda):
    net, info, hidden = _setup(cuda, torch.float32, 5)
    dec = BeliefDecoder(net, info, hidden)
    a = dec.sample(8, generator=torch.Generator(device=cuda).manual_seed(9))
    b = dec.sample(8, generator=torch.Generator(device=cuda).manual_seed(9))
    assert torch.equal(a, b)
    with pytest.raises(ValueError):
        dec.sample(41)
