"""The allocate-nothing fused layer (``atx_mha_fwd_noalloc``) against the
workspace entry point it varies (``atx_mha_fwd_ws``), through the C ABI.

The allocate-nothing call rearranges the weights into the library's own
per-GPU device array instead of a caller's workspace, then runs the same
kernel, so its output must equal ``atx_mha_fwd_ws``'s bit for bit.  Two calls
follow each other on one stream, the second on a smaller layer (fewer heads,
shorter sequence, smaller batch): the array keeps the first call's larger
contents, which the second must not read.
"""

from __future__ import annotations

import sys

import pytest
import torch

from ataraxos_amd import _lib, ops
from tests._cases import randn

pytestmark = pytest.mark.gpu


def _announce(msg: str) -> None:
    print(f"\n[case] {msg}", flush=True)
    sys.stdout.flush()


def _layer(e, seed, bias):
    g = torch.Generator().manual_seed(seed)
    ws = [((torch.rand(e, e, generator=g) * 2 - 1) * e**-0.5).bfloat16() for _ in range(4)]
    bs = [((torch.rand(e, generator=g) * 2 - 1) * e**-0.5).bfloat16() for _ in range(4)] if bias else [None] * 4
    return ws, bs


def test_noalloc_equals_the_workspace_entry_point(cuda):
    cases = [(16, 100, 8, False, True), (4, 40, 4, True, False)]  # second: smaller in every size
    got, want = [], []
    for b, l, h, causal, bias in cases:
        e = 64 * h
        _announce(f"noalloc b={b} l={l} h={h} causal={causal} bias={bias}")
        x = randn((b, l, e), 900 + h, torch.bfloat16).to(cuda)
        ws, bs = _layer(e, 901 + h, bias)
        wd = [w.to(cuda) for w in ws]
        bd = [t.to(cuda) if t is not None else None for t in bs]
        kw = dict(num_heads=h, b_q=bd[0], b_k=bd[1], b_v=bd[2], b_o=bd[3], causal=causal)
        got.append(ops.mha_forward(x, *wd, noalloc=True, **kw))
        want.append(ops.mha_forward(x, *wd, repack=True, **kw))
    torch.cuda.synchronize()
    for (b, l, h, _, _), g, w in zip(cases, got, want):
        assert torch.isfinite(g.float()).all()
        assert torch.equal(g, w), (b, l, h)


def test_noalloc_refuses_a_layer_beyond_its_array(cuda):
    p = _lib.MhaParams()
    p.abi_version, p.dtype, p.batch, p.seq, p.embed_dim, p.num_heads = _lib.ABI_VERSION, _lib.DTYPE_BF16, 2, 16, 640, 10
    p.x = p.w_q = p.w_k = p.w_v = p.w_o = p.y = 1 << 20  # never dereferenced: refused first
    p.x_stride_b = p.y_stride_b = 16 * 640
    p.x_stride_s = p.y_stride_s = 640
    p.scale = 0.125
    assert _lib.call("atx_mha_fwd_noalloc", p, None) == _lib.ERR_UNSUPPORTED
    assert "scratch" in _lib.last_error()
