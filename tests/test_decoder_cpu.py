"""use_hip_attention on the CPU: an in-place conversion that keeps the
parameters, state_dict and (CPU) results of ``nn.MultiheadAttention``."""

from __future__ import annotations

import copy

import pytest
import torch
import torch.nn as nn

from ataraxos_amd import KernelMultiheadAttention, use_hip_attention
from tests._netlike import belief_decoder


def test_conversion_keeps_state_and_cpu_results():
    torch.manual_seed(0)
    dec = belief_decoder(dim=64, heads=4, ff=128).eval()
    ref = copy.deepcopy(dec)
    keys = list(dec.state_dict())
    use_hip_attention(dec)
    kinds = [type(m) for m in dec.modules() if isinstance(m, nn.MultiheadAttention)]
    assert kinds and all(k is KernelMultiheadAttention for k in kinds)
    assert list(dec.state_dict()) == keys
    tgt, mem = torch.randn(3, 10, 64), torch.randn(3, 20, 64)
    mask = torch.triu(torch.full((10, 10), float("-inf")), 1)
    pad = torch.rand(3, 20) < 0.3
    pad[:, 0] = False
    want = ref(tgt, mem, tgt_mask=mask, memory_key_padding_mask=pad)
    got = dec(tgt, mem, tgt_mask=mask, memory_key_padding_mask=pad)
    assert torch.equal(got, want)


def test_unsupported_options_are_refused():
    with pytest.raises(NotImplementedError, match="add_bias_kv"):
        use_hip_attention(nn.MultiheadAttention(64, 4, add_bias_kv=True))
    with pytest.raises(NotImplementedError, match="head_dim"):
        use_hip_attention(nn.MultiheadAttention(64, 8))
