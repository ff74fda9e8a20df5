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


@pytest.mark.parametrize("dtype,tol,b", [(torch.float32, 1e-4, 16), (torch.bfloat16, 3e-2, 16), (torch.bfloat16, 3e-2, 2048)])
def test_belief_decoder_matches_torch(cuda, dtype, tol, b):
    """The reference's decoder stack -- 4 layers, dim 512, 8 heads, ff 2048
    (belief_net.py:105-114, constants.py:156-159) -- with the causal tgt_mask
    and memory_key_padding_mask = ~hidden_mask of belief_net.py:159-177, at
    B=16 and at config 4's B=2048, against torch's own module in fp32."""
    _announce(f"belief decoder {dtype} b={b}")
    torch.manual_seed(0)
    dec = belief_decoder(ff=2048, layers=4).eval()
    ref = copy.deepcopy(dec).to(cuda, dtype)
    dec = use_hip_attention(dec).to(cuda, dtype)
    s = 40
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


def test_decoder_self_attention_takes_the_fused_layer(cuda, monkeypatch):
    """In inference, TransformerDecoderLayer's self-attention (self_attn(x, x, x),
    causal hint, 8 heads x 64, 40 tokens) runs as one launch of the fused
    layer from the in_proj slices (rearranged on every call); it equals the projections +
    attention kernel path to bf16 rounding and the row-major fused call
    bit for bit.  With a key padding mask it keeps the unfused path."""
    from ataraxos_amd import ops
    import ataraxos_amd.decoder as dec_mod

    _announce("decoder self-attention fused")
    torch.manual_seed(3)
    m = use_hip_attention(torch.nn.MultiheadAttention(512, 8, batch_first=True)).to(cuda, torch.bfloat16).eval()
    x = torch.randn(6, 40, 512, device=cuda).bfloat16()
    calls = []
    real = ops.mha_forward
    monkeypatch.setattr(dec_mod.ops, "mha_forward", lambda *a, **k: calls.append(k.get("repack")) or real(*a, **k))
    with torch.no_grad():
        fused, _ = m(x, x, x, need_weights=False, is_causal=True, attn_mask=torch.zeros(40, 40, device=cuda))
        assert calls == [True]
        w_q, w_k, w_v = m.in_proj_weight.chunk(3)
        b_q, b_k, b_v = m.in_proj_bias.chunk(3)
        direct = real(x, w_q, w_k, w_v, m.out_proj.weight, num_heads=8, b_q=b_q, b_k=b_k, b_v=b_v,
                      b_o=m.out_proj.bias, causal=True)
        m.fuse_layer = False
        unfused, _ = m(x, x, x, need_weights=False, is_causal=True, attn_mask=torch.zeros(40, 40, device=cuda))
        m.fuse_layer = True
        pad = torch.zeros(6, 40, dtype=torch.bool, device=cuda)
        padded, _ = m(x, x, x, need_weights=False, key_padding_mask=pad)
    assert calls == [True]  # neither fuse_layer=False nor the padded call went fused
    assert torch.equal(fused, direct)
    assert _rel(fused, unfused) <= 2e-2
    assert torch.isfinite(padded.float()).all()


def test_decoder_self_attention_fused_sequence_first(cuda):
    """batch_first=False: the fused layer reads the [S, B, E] input through a
    transposed view and the result matches the batch-first module's."""
    _announce("decoder self-attention fused, sequence first")
    torch.manual_seed(4)
    mb = use_hip_attention(torch.nn.MultiheadAttention(384, 6, batch_first=True)).to(cuda, torch.bfloat16).eval()
    ms = use_hip_attention(torch.nn.MultiheadAttention(384, 6, batch_first=False)).to(cuda, torch.bfloat16).eval()
    ms.load_state_dict(mb.state_dict())
    x = torch.randn(5, 48, 384, device=cuda).bfloat16()
    xs = x.transpose(0, 1).contiguous()
    with torch.no_grad():
        yb, _ = mb(x, x, x, need_weights=False)
        ys, _ = ms(xs, xs, xs, need_weights=False)
    assert ys.shape == (48, 5, 384)
    assert torch.equal(ys.transpose(0, 1), yb)


def test_decoder_attention_dropout_in_the_kernel(cuda):
    """Training with the Belief decoder's dropout 0.2 (512 / 8 = head_dim 64):
    the converted cross-attention drops weights in the kernel; its output is
    nn.MultiheadAttention's math with the kernel's mask made explicit (fp32),
    repeatable under the same torch seed, and differentiable."""
    from ataraxos_amd import ops

    _announce("decoder cross-attention with dropout 0.2 in training")
    torch.manual_seed(0)
    m = use_hip_attention(torch.nn.MultiheadAttention(512, 8, dropout=0.2, batch_first=True)).to(cuda).train()
    b, sq, skv = 4, 40, 100
    q = torch.randn(b, sq, 512, device=cuda, requires_grad=True)
    kv = torch.randn(b, skv, 512, device=cuda)
    pad = torch.rand(b, skv, device=cuda) < 0.3
    pad[:, 0] = False
    torch.manual_seed(7)
    seed = ops.new_dropout_seed()
    torch.manual_seed(7)
    out, _ = m(q, kv, kv, key_padding_mask=pad, need_weights=False)
    torch.manual_seed(7)
    again, _ = m(q, kv, kv, key_padding_mask=pad, need_weights=False)
    assert torch.equal(out, again)
    # nn.MultiheadAttention's math with the kernel's keep decisions
    w_q, w_k, w_v = m.in_proj_weight.chunk(3)
    b_q, b_k, b_v = m.in_proj_bias.chunk(3)
    qh = torch.nn.functional.linear(q, w_q, b_q).view(b, sq, 8, 64).transpose(1, 2)
    kh = torch.nn.functional.linear(kv, w_k, b_k).view(b, skv, 8, 64).transpose(1, 2)
    vh = torch.nn.functional.linear(kv, w_v, b_v).view(b, skv, 8, 64).transpose(1, 2)
    s = torch.matmul(qh, kh.transpose(-1, -2).contiguous()) / 8.0
    s = s.masked_fill(pad[:, None, None, :], float("-inf"))
    keep = ops.dropout_mask(b, 8, sq, skv, 0.2, seed, device=cuda).float()
    scale = 1.0 / (1.0 - torch.tensor(0.2, dtype=torch.float32).item())
    p = torch.softmax(s, dim=-1) * keep * scale
    want = m.out_proj(torch.matmul(p, vh).transpose(1, 2).reshape(b, sq, 512))
    assert _rel(out, want) <= 1e-5
    out.sum().backward()
    assert q.grad is not None and torch.isfinite(q.grad).all()
    # eval: no dropout, deterministic without a seed
    m.eval()
    with torch.no_grad():
        e1, _ = m(q, kv, kv, key_padding_mask=pad, need_weights=False)
        e2, _ = m(q, kv, kv, key_padding_mask=pad, need_weights=False)
    assert torch.equal(e1, e2)
