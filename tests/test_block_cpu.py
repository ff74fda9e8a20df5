"""The drop-in pre-LN blocks on the CPU: the reference's submodule names,
state_dict keys and parameter creation order
(stratego/networks/transformer.py:107-124, 163-171), and the forward as the
reference composes it (:143-144) -- on the CPU the fused half never applies."""

from __future__ import annotations

import torch
import torch.nn as nn

from ataraxos_amd import MultiHeadAttention, PreLNTransformerBlock, TransformerStack

REF_KEYS = [
    "ln1.weight", "ln1.bias",
    "attn.q_proj.weight", "attn.k_proj.weight", "attn.v_proj.weight", "attn.out_proj.weight",
    "ln2.weight", "ln2.bias",
    "ff.0.weight", "ff.0.bias", "ff.2.weight", "ff.2.bias",
]


def test_state_dict_keys_and_creation_order():
    torch.manual_seed(0)
    blk = PreLNTransformerBlock(64, 4, 128)
    assert list(blk.state_dict().keys()) == REF_KEYS
    # the same draws as creating the reference's submodules in its order
    torch.manual_seed(0)
    ln1 = nn.LayerNorm(64)
    attn = MultiHeadAttention(64, 4)
    ln2 = nn.LayerNorm(64)
    ff = nn.Sequential(nn.Linear(64, 128), nn.GELU(), nn.Linear(128, 64))
    for a, b in zip(blk.parameters(), [*ln1.parameters(), *attn.parameters(), *ln2.parameters(), *ff.parameters()]):
        assert torch.equal(a, b)
    assert isinstance(blk.dropout, nn.Identity)
    assert isinstance(PreLNTransformerBlock(64, 4, 128, dropout=0.1).dropout, nn.Dropout)
    stack = TransformerStack(2, 64, 4, 128)
    assert list(stack.state_dict().keys()) == [f"blocks.{i}.{k}" for i in range(2) for k in REF_KEYS]


def test_forward_is_the_reference_composition():
    torch.manual_seed(1)
    blk = PreLNTransformerBlock(96, 3, 192, causal=True).eval()
    x = torch.randn(2, 11, 96)
    with torch.no_grad():
        ref = x + blk.attn(blk.ln1(x))
        ref = ref + blk.ff(blk.ln2(ref))
        assert torch.equal(blk(x), ref)
        kv = torch.randn(2, 5, 96)
        ref2 = x + blk.attn(blk.ln1(x), kv)
        ref2 = ref2 + blk.ff(blk.ln2(ref2))
        assert torch.equal(blk(x, kv), ref2)
    stack = TransformerStack(2, 96, 3, 192).eval()
    with torch.no_grad():
        assert torch.equal(stack(x), stack.blocks[1](stack.blocks[0](x)))
