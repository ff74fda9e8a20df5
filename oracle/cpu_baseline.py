"""CPU baseline: the reference's math path run with torch on the host CPU.

Test/bench infrastructure only (see ``oracle/__init__.py``): ``bench.py``
times these functions on the GPU box's host cores and reports the result as
``cpu_baseline`` (kind ``"port"``).  They restate, with the same torch calls
the reference makes on a CPU device,

* ``MultiHeadAttention._forward_math`` (stratego/networks/attention.py:281-316):
  BHSD transpose, ``matmul(q, k^T) * scale``, optional top-left causal
  ``-inf`` mask, ``softmax``, ``matmul(P, V)``, transpose back;
* ``KeyQueryPolicyHead`` logits/mask (stratego/networks/move_net.py:92-95) and
  the callers' softmax (stratego/training/selfplay.py:284).

Inputs are fp32 (the reference's CPU dtype) holding bf16-rounded values.
"""

from __future__ import annotations

import math
import os
import statistics
import time

import torch


def math_attention_cpu(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False) -> torch.Tensor:
    """BSHD in, BSHD out (H_kv == H), fp32 on the CPU."""
    qh, kh, vh = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    w = torch.matmul(qh, kh.transpose(-2, -1)) * (1.0 / math.sqrt(q.shape[-1]))
    if causal:
        w = w.masked_fill(torch.ones(q.shape[1], k.shape[1], dtype=torch.bool).triu(1), float("-inf"))
    w = torch.softmax(w, dim=-1)
    return torch.matmul(w, vh).transpose(1, 2)


def kq_probs_cpu(q: torch.Tensor, k: torch.Tensor, mask: torch.Tensor, scale: float) -> torch.Tensor:
    logits = torch.matmul(q, k.transpose(-2, -1)) * scale
    logits = logits.masked_fill(~mask, -1e10)
    return torch.softmax(logits.reshape(logits.shape[0], -1), dim=-1)


def cpu_info() -> dict:
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads()}


def time_fn(fn, warmup: int = 3, reps: int = 10, budget_s: float = 20.0) -> tuple[float, int]:
    """Median wall time of ``fn()`` over up to ``reps`` runs after ``warmup``,
    stopping early once ``budget_s`` seconds have been spent; returns
    (median seconds, runs timed)."""
    for _ in range(warmup):
        fn()
    times: list[float] = []
    start = time.perf_counter()
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - start > budget_s and len(times) >= 3:
            break
    return statistics.median(times), len(times)


def attention_baseline(batch: int, seq: int, heads: int, head_dim: int, threads: int, seed: int = 45) -> dict:
    """Time the math path on a ``[batch, seq, heads, head_dim]`` sample."""
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(seed)
    shape = (batch, seq, heads, head_dim)
    q, k, v = (torch.randn(shape, generator=g).bfloat16().float() for _ in range(3))
    with torch.inference_mode():
        t, runs = time_fn(lambda: math_attention_cpu(q, k, v))
    return {"seconds_per_call": t, "samples_per_s": batch / t, "runs": runs, **cpu_info()}


def kq_baseline(batch: int, seq: int, dim: int, threads: int, seed: int = 44) -> dict:
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, seq, dim, generator=g).bfloat16().float()
    k = torch.randn(batch, seq, dim, generator=g).bfloat16().float()
    mask = torch.rand(batch, seq, seq, generator=g) < 0.02
    mask[:, 0, 0] |= ~mask.flatten(1).any(dim=1)  # >= 1 legal entry per sample (config 2)
    with torch.inference_mode():
        t, runs = time_fn(lambda: kq_probs_cpu(q, k, mask, 1.0 / math.sqrt(dim)))
    return {"seconds_per_call": t, "samples_per_s": batch / t, "runs": runs, **cpu_info()}
