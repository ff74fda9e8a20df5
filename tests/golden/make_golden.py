"""Write the golden fixtures under ``tests/golden/`` from the float64 oracle.

The reference holds no golden values for this path (its tests check
invariants only), so the fixtures come from ``oracle/`` — which the CPU suite
pins independently (torch SDPA / nn.MultiheadAttention in float64, scipy,
closed forms).  They freeze those answers so that the GPU kernels and any
later change of the oracle are checked against the same numbers.

Inputs are drawn from seeded CPU generators and rounded to bf16 (stored as
raw uint16 bit patterns) unless the case is fp32; outputs are stored as
float32.  Run: ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle.attention import attention  # noqa: E402
from oracle.decode import decode_step  # noqa: E402
from oracle.policy import kq_logits, kq_probs  # noqa: E402

# name: (batch, seq_q, seq_kv, heads, kv_heads, head_dim, dtype, causal, pad_p)
ATTN_CASES = {
    "move_l100_bf16": (1, 100, 100, 2, 2, 64, "bf16", False, None),
    "move_l101_d48_bf16": (1, 101, 101, 2, 2, 48, "bf16", False, None),
    "setup_causal40_bf16": (2, 40, 40, 1, 1, 64, "bf16", True, None),
    "belief_cross_kpad_bf16": (2, 40, 100, 1, 1, 64, "bf16", False, 0.5),
    "gqa_8x2_fp32": (2, 33, 33, 8, 2, 32, "fp32", False, None),
    "causal_rect_fp32": (1, 10, 30, 4, 4, 16, "fp32", True, None),
    "long256_bf16": (1, 256, 256, 1, 1, 32, "bf16", False, None),
}


def draw(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(shape, generator=g)
    return t.bfloat16() if dtype == "bf16" else t


def pack(t: torch.Tensor) -> np.ndarray:
    """bf16 -> raw uint16 bits; fp32 stays float32."""
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy().astype(np.float32)


def unpack(a: np.ndarray) -> np.ndarray:
    """Inverse of :func:`pack`, as float64."""
    if a.dtype == np.uint16:
        return (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return a.astype(np.float64)


def make_attention() -> dict:
    out = {}
    for i, (name, (b, sq, skv, h, hkv, d, dt, causal, pad_p)) in enumerate(ATTN_CASES.items()):
        seed = 1000 + 10 * i
        q, k, v = draw((b, sq, h, d), seed, dt), draw((b, skv, hkv, d), seed + 1, dt), draw((b, skv, hkv, d), seed + 2, dt)
        pad = None
        if pad_p is not None:
            g = torch.Generator().manual_seed(seed + 3)
            pad = (torch.rand(b, skv, generator=g) < pad_p).numpy()
            pad[:, 0] = False  # every row keeps a key
        ref = attention(unpack(pack(q)), unpack(pack(k)), unpack(pack(v)), causal=causal, key_pad=pad)
        out[f"{name}/q"], out[f"{name}/k"], out[f"{name}/v"] = pack(q), pack(k), pack(v)
        out[f"{name}/o"] = ref.astype(np.float32)
        out[f"{name}/meta"] = np.array([b, sq, skv, h, hkv, d, int(causal), int(pad is not None)], dtype=np.int64)
        if pad is not None:
            out[f"{name}/key_pad"] = pad
    return out


def make_policy() -> dict:
    b, s, d = 4, 100, 64
    q, k = draw((b, s, d), 2000, "bf16"), draw((b, s, d), 2001, "bf16")
    g = torch.Generator().manual_seed(2002)
    mask = (torch.rand(b, s, s, generator=g) < 0.05).numpy()
    mask[3] = False
    mask[3, 42, 17] = True  # a sample with a single legal move
    scale = 1.0 / np.sqrt(d)
    qn, kn = unpack(pack(q)), unpack(pack(k))
    return {
        "q": pack(q),
        "k": pack(k),
        "mask": mask,
        "probs": kq_probs(qn, kn, mask, scale).astype(np.float32),
        "logits": kq_logits(qn, kn, mask, scale).astype(np.float32),
    }


def make_decode() -> dict:
    b, h, d, t = 2, 4, 64, 40
    q = draw((b, h, d), 3000, "bf16")
    kc = draw((b, h, t, d), 3001, "bf16")
    vc = draw((b, h, t, d), 3002, "bf16")
    steps = np.stack([decode_step(unpack(pack(q)), unpack(pack(kc))[:, :, :n], unpack(pack(vc))[:, :, :n]) for n in (1, 2, 17, 40)])
    return {"q": pack(q), "k_cache": pack(kc), "v_cache": pack(vc), "lens": np.array([1, 2, 17, 40]), "o": steps.astype(np.float32)}


def main() -> None:
    np.savez_compressed(HERE / "attention_cases.npz", **make_attention())
    np.savez_compressed(HERE / "policy_cases.npz", **make_policy())
    np.savez_compressed(HERE / "decode_cases.npz", **make_decode())
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main()
