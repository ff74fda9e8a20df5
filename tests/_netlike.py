"""Small modules with the reference networks' structure, for tests only.

``SetupLike`` mirrors ``SetupNetwork`` (``stratego/networks/setup_net.py:80-123``):
token + learned positional embedding, pre-LN causal blocks
(``stratego/networks/transformer.py:117-145``), value / entropy heads on
position 0 and a per-position policy head (``transformer.py:193-290``).
``belief_decoder`` builds the Belief network's decoder stack
(``stratego/networks/belief_net.py:105-114``).
"""

from __future__ import annotations

import torch
import torch.nn as nn

from ataraxos_amd import MultiHeadAttention


class _PosEmb(nn.Module):
    def __init__(self, max_len: int, dim: int) -> None:
        super().__init__()
        self.embed = nn.Parameter(torch.randn(max_len, dim) * 0.1)


class _Block(nn.Module):
    def __init__(self, dim: int, heads: int, ff: int) -> None:
        super().__init__()
        self.ln1 = nn.LayerNorm(dim)
        self.attn = MultiHeadAttention(dim, heads, causal=True)
        self.ln2 = nn.LayerNorm(dim)
        self.ff = nn.Sequential(nn.Linear(dim, ff), nn.GELU(), nn.Linear(ff, dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(self.ln1(x))
        return x + self.ff(self.ln2(x))


class _Stack(nn.Module):
    def __init__(self, depth: int, dim: int, heads: int, ff: int) -> None:
        super().__init__()
        self.blocks = nn.ModuleList([_Block(dim, heads, ff) for _ in range(depth)])


class _Head(nn.Module):
    def __init__(self, dim: int, out: int, first: bool) -> None:
        super().__init__()
        self.ln = nn.LayerNorm(dim)
        self.proj = nn.Linear(dim, out)
        self.first = first

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.first and x.dim() == 3:
            x = x[:, 0]
        return self.proj(self.ln(x))


class SetupLike(nn.Module):
    def __init__(self, depth: int = 4, dim: int = 512, heads: int = 8, ff: int = 1024, types: int = 12) -> None:
        super().__init__()
        self.token_emb = nn.Embedding(types, dim)
        self.pos_emb = _PosEmb(40, dim)
        self.blocks = _Stack(depth, dim, heads, ff)
        self.value_head = _Head(dim, 3, True)
        self.entropy_head = _Head(dim, 1, True)
        self.policy_head = _Head(dim, types, False)

    def forward(self, tokens: torch.Tensor):
        x = self.token_emb(tokens) + self.pos_emb.embed[: tokens.shape[1]]
        for blk in self.blocks.blocks:
            x = blk(x)
        return self.value_head(x), self.entropy_head(x), self.policy_head(x)


def belief_decoder(dim: int = 512, heads: int = 8, ff: int = 1024, layers: int = 2) -> nn.TransformerDecoder:
    layer = nn.TransformerDecoderLayer(d_model=dim, nhead=heads, dim_feedforward=ff, dropout=0.2,
                                       activation="gelu", norm_first=True, batch_first=True)
    return nn.TransformerDecoder(layer, num_layers=layers)


class _EncBlock(nn.Module):
    def __init__(self, dim: int, heads: int, ff: int) -> None:
        super().__init__()
        self.ln1 = nn.LayerNorm(dim)
        self.attn = MultiHeadAttention(dim, heads, causal=False)
        self.ln2 = nn.LayerNorm(dim)
        self.ff = nn.Sequential(nn.Linear(dim, ff), nn.GELU(), nn.Linear(ff, dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(self.ln1(x))
        return x + self.ff(self.ln2(x))


class BeliefLike(nn.Module):
    """The Belief network's structure (``stratego/networks/belief_net.py:67-180``):
    input projection + positional embedding + bidirectional encoder, token and
    positional embeddings, ``nn.TransformerDecoder`` (norm_first, gelu) with
    causal self-attention and key-padded cross-attention, output projection."""

    def __init__(self, channels: int = 32, dim: int = 256, heads: int = 4, ff: int = 512, enc_depth: int = 2,
                 dec_layers: int = 2, types: int = 12) -> None:
        super().__init__()
        self.input_proj = nn.Linear(channels, dim)
        self.enc_pos_emb = _PosEmb(100, dim)
        self.encoder = nn.ModuleList([_EncBlock(dim, heads, ff) for _ in range(enc_depth)])
        self.token_emb = nn.Embedding(types, dim)
        self.dec_pos_emb = _PosEmb(40, dim)
        self.decoder = belief_decoder(dim, heads, ff, dec_layers)
        self.output_proj = nn.Linear(dim, types)

    def forward(self, infostate: torch.Tensor, hidden_mask: torch.Tensor, target_tokens: torch.Tensor | None = None):
        x = self.input_proj(infostate.permute(0, 2, 3, 1).flatten(1, 2)) + self.enc_pos_emb.embed
        for blk in self.encoder:
            x = blk(x)
        if target_tokens is None:
            return x
        s = target_tokens.shape[1]
        tgt = self.token_emb(target_tokens) + self.dec_pos_emb.embed[:s]
        mask = torch.triu(torch.full((s, s), float("-inf"), device=tgt.device, dtype=tgt.dtype), diagonal=1)
        out = self.decoder(tgt, x, tgt_mask=mask, memory_key_padding_mask=~hidden_mask)
        return self.output_proj(out)
