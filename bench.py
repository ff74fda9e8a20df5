"""Benchmark of the attention hot path on one MI355X (gfx950).

Workload: the Move-network encoder attention stack at the
self-play inference batch — B=4096, L=100, E=384, 6 heads x 64, bf16, 8
consecutive bidirectional self-attention layers.  Each layer's Q/K/V come from
a seeded N(0, 0.02) random-init projection of N(0, 1) tokens and are resident
in HBM before timing starts (8 layers x 3 x 315 MB).

A step is one pass of the fused HIP attention kernel over all 8 layers.
``value`` is samples/s through one attention layer (8*B / step time), the
unit in which the north-star target is stated (>= 70 % of the 8 TB/s HBM
roofline = 18.2 M samples/s).  Also reported on the same line:

* ``roofline`` for the attention kernel: algorithmic bytes per launch
  (B x 307,200 B: Q, K, V read + O written in bf16) over the kernel's mean
  duration, measured with events recorded on the launch stream around every
  launch in the timed region; ``traffic`` is the HBM bytes per launch read
  from the committed rocprofv3 counter summary when present;
* ``mfma``: the same kernel's algorithmic FLOP rate (B x 15.36 MFLOP) against
  the 2.5 PFLOP/s dense bf16 peak;
* ``e2e``: the full MultiHeadAttention forward of the 8 layers plus the
  residual, as the module runs it in inference (one launch of the fused layer
  kernel per layer), with its MFMA rate (B x 133.3 MFLOP per layer), and the
  same with the unfused path (hipBLASLt projections + attention kernel); the
  chain with the residual inside the layer kernel; the attention halves of 8
  pre-LN blocks (LayerNorm + layer + residual, one launch each); one layer of
  the reference Move network's 8 x 48 at L=101;
* ``kq_policy``: the fused key-query policy kernel at config C2;
* ``belief_attention``: the attention kernel at the config C4 shapes
  (encoder self, decoder causal self, decoder cross with key padding);
* ``decode``: the KV-cache decode kernel over config C5's 4 layers x 40 steps;
* ``backward``: the attention backward kernel (dQ, dK, dV) of one C3 layer;
* ``kq_backward``: the policy-head backward kernel (dq, dk) at config C2;
* ``rollout``: the self-play producer (HIP Stratego simulator) at 4096 games:
  legal-move mask and infostate kernels against the HBM roofline, one ply;
* ``cpu_baseline``: the reference's math path (torch on the host CPU) on a
  bounded sample of the same layer, rank 0 only.

``python bench.py --gpus N --steps K --warmup W``; only N=1 is supported.

Warm-up: after an idle spell the MI355X needs about 80-100 ms of continuous
work before a launch reaches its steady duration (a C4 encoder launch went
from 190 us to 148 us over the first 100 ms).  The default 60 warm-up steps
of the main leg are ~100 ms; every other leg first runs its own launches
untimed for at least ``SETTLE_MS``.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "Move-net attn fwd samples/s @B=4096,L=100 bf16; % of bf16 MFMA peak"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6
FP32_PEAK_TFLOPS = 157.3  # dense fp32 MFMA
TRAFFIC_FILE = ROOT / "profiles" / "attn_fwd_c3_traffic.json"
SETTLE_MS = 150.0


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=60)
    ap.add_argument("--batch", type=int, default=4096)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--qkv", choices=("separate", "packed"), default="separate",
                    help="q/k/v as three tensors or as views of one fused [B, L, 3E] projection")
    ap.add_argument("--no-extras", action="store_true", help="skip the e2e, kq_policy, belief_attention, decode, backward and rollout legs")
    ap.add_argument("--cpu-sample", type=int, default=4096, help="batch of the C3 CPU baseline sample")
    ap.add_argument(
        "--mode",
        choices=("bench", "pmc"),
        default="bench",
        help="pmc: only launch one kernel (--pmc-kernel) `steps` times and a 1 GiB plain copy `steps` "
        "times (the calibration for rocprofv3 FETCH_SIZE / WRITE_SIZE passes); prints no JSON",
    )
    ap.add_argument("--pmc-kernel", choices=("attn_fwd", "attn_bwd", "kq_bwd", "mha", "rollout"), default="attn_fwd",
                    help="pmc mode: the C3 attention forward, its backward, the C2 policy backward (logits), "
                    "the fused C3 layer, or the simulator's infostate + legal-mask kernels at 4096 games")
    return ap.parse_args()


def pmc_workload(torch, ops, batch, steps, dev, kernel="attn_fwd") -> None:
    """One C3 layer through the chosen kernel `steps` times, then a plain
    device copy of exactly 1 GiB (read 1 GiB + write 1 GiB) to scale the byte
    counters."""
    if kernel == "rollout":
        from ataraxos_amd import StrategoRolloutBuffer

        buf, _ = _rollout_midgame(torch, dev, batch)
        mask = torch.empty(batch, 100, 100, dtype=torch.bool, device=dev)
        info = torch.empty(batch, 488, 10, 10, dtype=torch.float32, device=dev)
        for _ in range(steps):
            buf.compute_infostate_tensor(out=info)
            buf.compute_legal_action_mask(out=mask)
        _copy_calibration(torch, steps, dev)
        print(f"[pmc] rollout infostate + mask x{steps} ({batch} games) and 1 GiB copy x{steps} done",
              file=sys.stderr, flush=True)
        return
    layers = make_layers(torch, batch, 100, 384, 1, dev)
    q, k, v = (t.view(batch, 100, 6, 64) for t in layers[0])
    out = torch.empty_like(q)
    if kernel == "attn_fwd":
        for _ in range(steps):
            ops.attention_forward(q, k, v, out=out)
    elif kernel == "attn_bwd":
        o = ops.attention_forward(q, k, v)
        for _ in range(steps):
            ops.attention_backward(q, k, v, o, o)
    elif kernel == "kq_bwd":
        g = torch.Generator(device=dev).manual_seed(49)
        qk, kk = q[:, :, 0], k[:, :, 0]  # [B, 100, 64] views
        mask = torch.rand(batch, 100, 100, generator=g, device=dev) < 0.02
        grad = torch.randn(batch, 100 * 100, generator=g, device=dev)
        for _ in range(steps):
            ops.kq_policy_backward(qk, kk, grad, mask)
    else:
        x = layers[0][0]
        ws = [(torch.randn(384, 384, device=dev) * 0.05).to(torch.bfloat16) for _ in range(4)]
        ws = [ops.mha_pack_weight(w) for w in ws]  # the order MultiHeadAttention's fused path reads
        y = torch.empty_like(x)
        for _ in range(steps):
            ops.mha_forward(x, *ws, num_heads=6, out=y, packed=True)
    _copy_calibration(torch, steps, dev)
    print(f"[pmc] {kernel} x{steps} (B={batch}) and 1 GiB copy x{steps} done", file=sys.stderr, flush=True)


def _copy_calibration(torch, steps, dev) -> None:
    torch.cuda.synchronize()
    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()


def make_layers(torch, batch, seq, embed, layers, dev, packed=False):
    """Per-layer resident (q, k, v), each [B, L, E].  ``packed``: one fused
    QKV projection per layer, q/k/v being strided views of its [B, L, 3E]
    output; otherwise three separate projections (three tensors)."""
    g = torch.Generator(device=dev).manual_seed(45)
    x = torch.randn(batch, seq, embed, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    out = []
    for _ in range(layers):
        w = [
            (torch.randn(embed, embed, generator=g, device=dev, dtype=torch.float32) * 0.02).to(torch.bfloat16)
            for _ in range(3)
        ]
        if packed:
            qkv = torch.matmul(x, torch.cat(w, dim=1))
            out.append((qkv[..., :embed], qkv[..., embed : 2 * embed], qkv[..., 2 * embed :]))
        else:
            out.append(tuple(torch.matmul(x, wi) for wi in w))
    del x
    return out


def time_attention(torch, ops, layers, heads, head_dim, steps, warmup):
    """Time `steps` passes over all layers after `warmup` untimed passes and
    at least ``SETTLE_MS`` of continuous untimed passes (the clocks' ramp, so
    the timed region sees the steady state whatever `warmup` is).  Returns
    (ms_per_step, per-launch kernel ms: mean, median, min)."""
    b, l, e = layers[0][0].shape
    views = [tuple(t.unflatten(-1, (heads, head_dim)) for t in qkv) for qkv in layers]
    outs = [torch.empty(b, l, heads, head_dim, dtype=torch.bfloat16, device=layers[0][0].device) for _ in layers]

    def one_pass():
        for (q, k, v), o in zip(views, outs):
            ops.attention_forward(q, k, v, out=o)

    for _ in range(warmup):
        one_pass()
    _settle(torch, one_pass)
    n = steps * len(views)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    i = 0
    for _ in range(steps):
        for (q, k, v), o in zip(views, outs):
            ev[i].record()
            ops.attention_forward(q, k, v, out=o)
            i += 1
    ev[i].record()
    stop.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(stop)
    per_launch = [ev[j].elapsed_time(ev[j + 1]) for j in range(n)]
    return total_ms / steps, sum(per_launch) / len(per_launch), statistics.median(per_launch), min(per_launch)


def time_e2e(torch, batch, seq, embed, heads, layers_n, steps, warmup, dev, fuse=True):
    """Full MHA forward x layers (x = x + mha(x)): with ``fuse`` each layer is
    one launch of the fused layer kernel; without, hipBLASLt projections +
    the attention kernel + hipBLASLt output projection."""
    from ataraxos_amd import MultiHeadAttention

    torch.manual_seed(45)
    mods = [MultiHeadAttention(embed, heads).to(dev, torch.bfloat16).eval() for _ in range(layers_n)]
    for m in mods:
        m.fuse_layer = fuse
    for m in mods:
        for p in m.parameters():
            torch.nn.init.normal_(p, std=0.02)
    g = torch.Generator(device=dev).manual_seed(45)
    x0 = torch.randn(batch, seq, embed, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)

    def step():
        x = x0
        for m in mods:
            x = x + m(x)
        return x

    with torch.inference_mode():
        for _ in range(warmup):
            step()
        _settle(torch, step)
        a, z = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            step()
        z.record()
        torch.cuda.synchronize()
    return a.elapsed_time(z) / steps


def time_chain(torch, ops, batch, seq, embed, heads, layers_n, steps, warmup, dev, ln=False, fuse=True):
    """The C3 chain with the residual inside the layer kernel: per layer one
    launch rearranging the weights and one launch computing x + MHA(x) (with
    ``ln``: x + MHA(LayerNorm(x)), the attention half of the reference's
    pre-LN block, transformer.py:143).  Without ``fuse`` the same chain as
    separate launches: LayerNorm (torch), the fused layer, the add."""
    g = torch.Generator(device=dev).manual_seed(47)
    x0 = torch.randn(batch, seq, embed, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    ws = [[(torch.randn(embed, embed, generator=g, device=dev) * 0.02).to(torch.bfloat16) for _ in range(4)]
          for _ in range(layers_n)]
    lns = [((1 + 0.1 * torch.randn(embed, generator=g, device=dev)).to(torch.bfloat16),
            (0.1 * torch.randn(embed, generator=g, device=dev)).to(torch.bfloat16)) for _ in range(layers_n)]
    work = torch.empty(ops.mha_workspace_bytes(embed), dtype=torch.uint8, device=dev)

    def step():
        x = x0
        for w, (lw, lb) in zip(ws, lns):
            if fuse:
                kw = dict(ln_weight=lw, ln_bias=lb) if ln else {}
                x = ops.mha_forward(x, *w, num_heads=heads, repack=True, workspace=work, residual=True, **kw)
            else:
                h = torch.nn.functional.layer_norm(x, (embed,), lw, lb, 1e-5) if ln else x
                x = x + ops.mha_forward(h, *w, num_heads=heads, repack=True, workspace=work)
        return x

    with torch.inference_mode():
        for _ in range(warmup):
            step()
        _settle(torch, step)
        a, z = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            step()
        z.record()
        torch.cuda.synchronize()
    return a.elapsed_time(z) / steps


def time_kq(torch, ops, batch, dev, steps, warmup):
    """Config C2: q, k [B, 100, 64] bf16, Bernoulli(0.02) legal mask, fp32 probs."""
    g = torch.Generator(device=dev).manual_seed(44)
    s, d = 100, 64
    q = torch.randn(batch, s, d, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(batch, s, d, generator=g, device=dev).to(torch.bfloat16)
    mask = torch.rand(batch, s, s, generator=g, device=dev) < 0.02
    mask[:, 0, 0] |= ~mask.flatten(1).any(dim=1)
    out = torch.empty(batch, s * s, dtype=torch.float32, device=dev)
    ms = _mean_launch_ms(torch, lambda: ops.kq_policy(q, k, mask, out=out), steps, warmup)
    bytes_per_sample = 2 * s * d * 2 + s * s + s * s * 4
    # the reference Move network's own head: 101 squares, d=384 (rows start at any alignment)
    s2, d2 = 101, 384
    q2 = torch.randn(batch, s2, d2, generator=g, device=dev).to(torch.bfloat16)
    k2 = torch.randn(batch, s2, d2, generator=g, device=dev).to(torch.bfloat16)
    m2 = torch.rand(batch, s2, s2, generator=g, device=dev) < 0.02
    m2[:, 0, 0] |= ~m2.flatten(1).any(dim=1)
    out2 = torch.empty(batch, s2 * s2, dtype=torch.float32, device=dev)
    ms2 = _mean_launch_ms(torch, lambda: ops.kq_policy(q2, k2, m2, out=out2), steps, warmup)
    bytes2 = 2 * s2 * d2 * 2 + s2 * s2 + s2 * s2 * 4
    return {
        "config": "C2 KQ logits + legal mask + softmax, B=4096, 100x100, d=64, bf16 in, fp32 out",
        "samples_per_s": batch / (ms * 1e-3),
        "kernel_ms": ms,
        "achieved_gbs": batch * bytes_per_sample / (ms * 1e-3) / 1e9,
        "hbm_frac": batch * bytes_per_sample / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "move_ref_d384": _leg("policy head forward (probabilities) at the reference Move head's shape "
                              "(B=4096, 101 squares, d=384), bf16", ms2, batch * bytes2, batch),
    }


def _settle(torch, fn, min_ms=SETTLE_MS):
    """Run ``fn()`` untimed, in bursts, until the GPU has been kept busy with
    it for at least ``min_ms`` of wall time, so that what follows is timed at
    the steady clocks."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 1
    while True:
        t1 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        now = time.perf_counter()
        if (now - t0) * 1e3 >= min_ms:
            return
        if (now - t1) * 1e3 < 20.0:
            n *= 2


def _mean_launch_ms(torch, fn, steps, warmup):
    """Mean time per call of ``fn()`` (one kernel launch) over ``steps``
    back-to-back calls, from one event pair around them, after ``warmup``
    calls and :func:`_settle`.  An untimed burst queued right before keeps the
    GPU busy while the host enqueues the timed calls, so host launch overhead
    of short kernels does not enter the time."""
    for _ in range(warmup):
        fn()
    _settle(torch, fn)
    for _ in range(max(warmup, 20)):
        fn()
    a, z = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        fn()
    z.record()
    torch.cuda.synchronize()
    return a.elapsed_time(z) / steps


def _leg(what, ms, nbytes, samples):
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"what": what, "kernel_us": ms * 1e3, "achieved_gbs": gbs, "hbm_frac": gbs / HBM_PEAK_GBS,
            "samples_per_s": samples / (ms * 1e-3)}


def time_belief(torch, ops, dev, steps, warmup):
    """Config C4 attention shapes, B=2048, 8 heads x 64, bf16: encoder
    self-attention (L=100), decoder causal self-attention (40 tokens), decoder
    cross-attention 40 -> 100 with all keys valid and with a Bernoulli(0.4)
    key-padding mask (>= 1 valid key per sample)."""
    g = torch.Generator(device=dev).manual_seed(46)
    b, h, d, e = 2048, 8, 64, 512

    def bshd(s):
        return torch.randn(b, s, e, generator=g, device=dev).to(torch.bfloat16).view(b, s, h, d)

    enc = [bshd(100) for _ in range(3)]
    dec = [bshd(40) for _ in range(3)]
    pad = torch.rand(b, 100, generator=g, device=dev) < 0.4
    pad[:, 0] &= pad[:, 1:].all(dim=1).logical_not()  # keep key 0 valid where all others are padded
    o100, o40 = torch.empty_like(enc[0]), torch.empty_like(dec[0])
    row = e * 2  # bytes of one token's Q, K, V or O row
    legs = {
        "encoder_self_L100": _leg(
            "encoder self-attention, S=100", _mean_launch_ms(torch, lambda: ops.attention_forward(*enc, out=o100), steps, warmup),
            b * 100 * row * 4, b),
        "decoder_self_causal_L40": _leg(
            "decoder causal self-attention, S=40",
            _mean_launch_ms(torch, lambda: ops.attention_forward(*dec, causal=True, out=o40), steps, warmup),
            b * 40 * row * 4, b),
        "decoder_cross_40x100": _leg(
            "decoder cross-attention 40 -> 100",
            _mean_launch_ms(torch, lambda: ops.attention_forward(dec[0], enc[1], enc[2], out=o40), steps, warmup),
            b * (40 * 2 + 100 * 2) * row, b),
        "decoder_cross_40x100_keypad": _leg(
            "decoder cross-attention 40 -> 100, Bernoulli(0.4) key padding",
            _mean_launch_ms(torch, lambda: ops.attention_forward(dec[0], enc[1], enc[2], key_padding_mask=pad, out=o40),
                            steps, warmup),
            b * (40 * 2 + 100 * 2) * row + b * 100, b),
    }
    total_us = 6 * legs["encoder_self_L100"]["kernel_us"] + 4 * (
        legs["decoder_self_causal_L40"]["kernel_us"] + legs["decoder_cross_40x100_keypad"]["kernel_us"])
    return {"config": "C4 Belief-net attention, B=2048, 8x64, bf16", "legs": legs,
            "attention_us_per_forward": total_us,
            "note": "attention_us_per_forward = 6 encoder layers + 4 decoder layers (causal self + padded cross)"}


def time_decode(torch, ops, dev, reps):
    """Config C5: B=8192, 8 heads x 64, bf16, 4 layers x 40 steps; step t
    appends the new K/V row to each layer's [B, 8, 40, 64] cache and attends
    over t rows.  Whole 160-launch sequence timed, ``reps`` times."""
    g = torch.Generator(device=dev).manual_seed(47)
    b, h, d, t_max, n_layers = 8192, 8, 64, 40, 4
    caches = [(torch.zeros(b, h, t_max, d, dtype=torch.bfloat16, device=dev),
               torch.zeros(b, h, t_max, d, dtype=torch.bfloat16, device=dev)) for _ in range(n_layers)]
    step_in = [tuple(torch.randn(b, h, d, generator=g, device=dev).to(torch.bfloat16) for _ in range(3))
               for _ in range(n_layers)]
    out = torch.empty(b, h, d, dtype=torch.bfloat16, device=dev)

    def sequence():
        for t in range(1, t_max + 1):
            for (kc, vc), (q, kn, vn) in zip(caches, step_in):
                ops.attention_decode(q, kc, vc, t, kn, vn, out=out)

    sequence()
    _settle(torch, sequence)
    a, z = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        sequence()
    z.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(z) / reps
    e = h * d
    # per layer-step: K/V rows 0..t-1 read (the new row from k_new / v_new),
    # the new rows written to the caches, q read, o written
    nbytes = sum(n_layers * (2 * b * h * t * d * 2 + 2 * b * e * 2 + 2 * b * e * 2) for t in range(1, t_max + 1))
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"config": "C5 Setup-net decode, B=8192, 8x64, bf16, 4 layers x 40 steps",
            "ms_per_sequence": ms, "launches": t_max * n_layers, "us_per_launch": ms * 1e3 / (t_max * n_layers),
            "achieved_gbs": gbs, "hbm_frac": gbs / HBM_PEAK_GBS, "bytes_per_sequence": nbytes}


def time_backward(torch, ops, batch, dev, steps, warmup):
    """Backward of the C3 attention layer (B=4096, L=100, 6 x 64, bf16): the
    gradient the Move trainer takes through attention.  Q, K, V, the forward
    output O and dO are resident; one launch writes dQ, dK, dV."""
    g = torch.Generator(device=dev).manual_seed(48)
    s, h, d = 100, 6, 64
    q, k, v, do = (torch.randn(batch, s, h, d, generator=g, device=dev).to(torch.bfloat16) for _ in range(4))
    o = ops.attention_forward(q, k, v)
    ms = _mean_launch_ms(torch, lambda: ops.attention_backward(q, k, v, o, do), steps, warmup)
    nbytes = batch * h * 8 * s * d * 2  # Q, K, V, O, dO read; dQ, dK, dV written
    flops = batch * h * 5 * 2 * s * s * d  # S recomputed, dP, dV, dQ, dK
    leg = _leg("attention backward, C3 layer", ms, nbytes, batch)
    leg.update({"config": "C3 layer backward, B=4096, L=100, 6x64, bf16", "kernel": "attn_bwd_16bit<bf16, D=64, NKC=4>",
                "algorithmic_bytes_per_launch": nbytes, "tflops": flops / (ms * 1e-3) / 1e12,
                "mfma_frac": flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS})
    # fp32 (what the reference's trainers run) and GQA 6/2 at the same shape
    q32, k32, v32, do32 = (t.float() for t in (q, k, v, do))
    o32 = ops.attention_forward(q32, k32, v32)
    ms32 = _mean_launch_ms(torch, lambda: ops.attention_backward(q32, k32, v32, o32, do32), max(5, steps // 5), 3)
    f = flops / (ms32 * 1e-3) / 1e12
    leg["fp32"] = _leg("attention backward, C3 layer, fp32", ms32, 2 * nbytes, batch)
    leg["fp32"].update({"kernel": "attn_bwd_fp32<D=64, NKC=4>", "tflops": f, "fp32_mfma_frac": f / FP32_PEAK_TFLOPS})
    kg, vg = k[:, :, :2].contiguous(), v[:, :, :2].contiguous()
    og = ops.attention_forward(q, kg, vg)
    msg = _mean_launch_ms(torch, lambda: ops.attention_backward(q, kg, vg, og, do), max(5, steps // 5), 3)
    gbytes = batch * s * d * 2 * (4 * h + 4 * 2)  # Q, O, dO, dQ per query head; K, V, dK, dV per KV head
    leg["gqa_6_2"] = _leg("attention backward, C3 layer with 2 KV heads (GQA 6/2), bf16", msg, gbytes, batch)
    return leg


def time_kq_backward(torch, ops, batch, dev, steps, warmup):
    """Backward of the C2 policy head (B=4096, 100x100, d=64, bf16 q/k): the
    gradient the Move trainer takes through the logits, and through the
    probabilities for a caller that differentiates those."""
    g = torch.Generator(device=dev).manual_seed(49)
    s, d = 100, 64
    q = torch.randn(batch, s, d, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(batch, s, d, generator=g, device=dev).to(torch.bfloat16)
    mask = torch.rand(batch, s, s, generator=g, device=dev) < 0.02
    mask[:, 0, 0] |= ~mask.flatten(1).any(dim=1)
    grad = torch.randn(batch, s * s, generator=g, device=dev)
    probs = ops.kq_policy(q, k, mask, output="probs")
    legs = {}
    for output in ("logits", "probs"):
        ms = _mean_launch_ms(
            torch, lambda: ops.kq_policy_backward(q, k, grad, mask, output=output, probs=probs), steps, warmup)
        # G (and P) fp32 + legality bytes + q, k read; dq, dk written
        nbytes = batch * (s * s * 4 * (2 if output == "probs" else 1) + s * s + 4 * s * d * 2)
        legs[output] = _leg(f"policy head backward, gradient of the {output}", ms, nbytes, batch)
    # fp32 q/k at C2, and the reference Move network's own head: 101 squares, d=384
    q32, k32 = q.float(), k.float()
    ms = _mean_launch_ms(torch, lambda: ops.kq_policy_backward(q32, k32, grad, mask), max(5, steps // 5), 3)
    legs["logits_fp32"] = _leg("policy head backward, gradient of the logits, fp32 q/k", ms,
                               batch * (s * s * 4 + s * s + 4 * s * d * 4), batch)
    s2, d2 = 101, 384
    q2 = torch.randn(batch, s2, d2, generator=g, device=dev).to(torch.bfloat16)
    k2 = torch.randn(batch, s2, d2, generator=g, device=dev).to(torch.bfloat16)
    m2 = torch.rand(batch, s2, s2, generator=g, device=dev) < 0.02
    g2 = torch.randn(batch, s2 * s2, generator=g, device=dev)
    ms = _mean_launch_ms(torch, lambda: ops.kq_policy_backward(q2, k2, g2, m2), max(5, steps // 5), 3)
    legs["logits_move_ref_d384"] = _leg("policy head backward at the reference Move head's shape (101 squares, d=384), bf16",
                                        ms, batch * (s2 * s2 * 4 + s2 * s2 + 4 * s2 * d2 * 2), batch)
    # the same head in fp32, the precision the reference's Move trainer runs it in
    q2f, k2f = q2.float(), k2.float()
    ms = _mean_launch_ms(torch, lambda: ops.kq_policy_backward(q2f, k2f, g2, m2), max(5, steps // 5), 3)
    legs["logits_move_ref_d384_fp32"] = _leg(
        "policy head backward at the reference Move head's shape (101 squares, d=384), fp32 q/k", ms,
        batch * (s2 * s2 * 4 + s2 * s2 + 4 * s2 * d2 * 4), batch)
    return {"config": "C2 policy head backward, B=4096, 100x100, d=64, bf16 q/k, fp32 gradient", "legs": legs}


def _rollout_midgame(torch, dev, n):
    """A simulator of ``n`` games from random full setups after 40 random
    legal plies (finished games restarted), and its (pick, setups) helpers:
    ``pick()`` draws one random legal action per game on the GPU."""
    from ataraxos_amd import StrategoRolloutBuffer

    g = torch.Generator(device=dev).manual_seed(50)
    counts = {1: 1, 2: 8, 3: 5, 4: 4, 5: 4, 6: 4, 7: 3, 8: 2, 9: 1, 10: 1, 11: 1, 12: 6}
    pieces = torch.tensor([p for p, k in counts.items() for _ in range(k)], dtype=torch.int8, device=dev)

    def setups():
        red = torch.zeros(n, 10, 10, dtype=torch.int8, device=dev)
        blue = torch.zeros_like(red)
        for grid, rows in ((red, slice(0, 4)), (blue, slice(6, 10))):
            perm = torch.argsort(torch.rand(n, 40, generator=g, device=dev), dim=1)
            grid[:, rows] = pieces[perm].view(n, 4, 10)
        return red, blue

    buf = StrategoRolloutBuffer(n, 0)
    buf.reset_all(*setups())
    scratch = torch.empty(n, 100, 100, dtype=torch.bool, device=dev)

    def pick():
        m = buf.compute_legal_action_mask(out=scratch).view(n, -1)
        a = torch.rand(n, 10000, generator=g, device=dev).masked_fill_(~m, -1.0).argmax(dim=1)
        return a.masked_fill_(~m.any(dim=1), -1)

    for ply in range(40):
        buf.apply_actions(pick())
        if ply % 10 == 9:
            buf.reset_terminated(*setups())
    return buf, (pick, setups)


def time_rollout(torch, dev, steps, warmup):
    """The self-play producer at the config-2 batch: 4096 games of the HIP
    Stratego simulator in mid-game positions (random full setups, 40 random
    legal plies).  Legal-move mask and infostate kernels as bursts against
    the HBM roofline; ``apply`` per launch (events around each launch) over
    ``steps`` plies of random legal play, finished games restarted."""
    n = 4096
    buf, play = _rollout_midgame(torch, dev, n)
    mask = torch.empty(n, 100, 100, dtype=torch.bool, device=dev)
    info = torch.empty(n, 488, 10, 10, dtype=torch.float32, device=dev)
    pick, setups = play
    ms_mask = _mean_launch_ms(torch, lambda: buf.compute_legal_action_mask(out=mask), steps, warmup)
    ms_info = _mean_launch_ms(torch, lambda: buf.compute_infostate_tensor(out=info), steps, warmup)
    ms_hash = _mean_launch_ms(torch, lambda: buf.hash_board(), steps, warmup)
    pairs = []
    for ply in range(steps):
        a = pick()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        buf.apply_actions(a)
        e1.record()
        pairs.append((e0, e1))
        if ply % 10 == 9:
            buf.reset_terminated(*setups())
    torch.cuda.synchronize()
    ms_apply = sum(a.elapsed_time(z) for a, z in pairs) / len(pairs)
    mask_bytes = 10000 + 200 + 1  # mask written; owner, piece, side to move read
    info_bytes = 488 * 100 * 4 + 400 + 32 * 4 + 13  # infostate written; board, flags, history, scalars read
    legs = {
        "legal_mask": _leg("legal-move mask [4096, 100, 100] bool", ms_mask, n * mask_bytes, n),
        "infostate": _leg("infostate [4096, 488, 10, 10] float32", ms_info, n * info_bytes, n),
        "apply": {"what": "apply_actions, one ply of random legal play", "kernel_us": ms_apply * 1e3,
                  "games_per_s": n / (ms_apply * 1e-3)},
        "hash": {"what": "Zobrist hash of every board", "kernel_us": ms_hash * 1e3},
    }
    step_ms = ms_mask + ms_info + ms_apply
    return {"config": "self-play producer, 4096 games (config 2's batch), mid-game positions", "legs": legs,
            "ply_us": step_ms * 1e3, "game_plies_per_s": n / (step_ms * 1e-3),
            "note": "ply_us = legal mask + infostate + apply: what the producer launches per ply"}


def cpu_baseline(sample: int) -> dict:
    """The reference's math path timed with torch on the host CPU (fp32 on
    bf16-rounded inputs, 3 warm-ups, median of <= 10 runs): C3 at the
    benchmark batch (``value``), C1 at B=64 and the C2 policy softmax at
    B=4096.  Threads: the box's CPU share (OMP_NUM_THREADS, 16 on the GPU
    boxes), capped by os.cpu_count()."""
    from oracle.cpu_baseline import attention_baseline, kq_baseline

    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    threads = min(threads, os.cpu_count() or threads)
    c3 = attention_baseline(sample, 100, 6, 64, threads)
    c1 = attention_baseline(64, 100, 6, 64, threads, seed=42)
    c2 = kq_baseline(4096, 100, 64, threads)

    def leg(r, what, batch, nbytes, flops):
        t = r["seconds_per_call"]
        return {"what": what, "batch": batch, "samples_per_s": batch / t, "ms_per_call": t * 1e3,
                "gbs": batch * nbytes / t / 1e9, "tflops": batch * flops / t / 1e12, "runs": r["runs"]}

    return {
        "value": c3["samples_per_s"],
        "unit": "samples/s",
        "cores": c3["torch_threads"],
        "kind": "port",
        "sample": f"C3 self-attention core, B={sample}, L=100, 6x64, torch fp32 math path on the host CPU",
        "cpu_model": c3["cpu_model"],
        "os_cpu_count": c3["os_cpu_count"],
        "torch_threads": c3["torch_threads"],
        "legs": {
            "C3": leg(c3, "attention core, B=%d, L=100, 6x64" % sample, sample, 4 * 100 * 384 * 4,
                      4 * 6 * 100 * 100 * 64),
            "C1": leg(c1, "attention core, B=64, L=100, 6x64 (config 1)", 64, 4 * 100 * 384 * 4, 4 * 6 * 100 * 100 * 64),
            "C2": leg(c2, "policy logits + legal mask + softmax over 10^4, B=4096, d=64", 4096,
                      2 * 100 * 64 * 4 + 100 * 100 + 100 * 100 * 4, 2 * 100 * 100 * 64),
        },
    }


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(
            f"bench.py: --gpus {args.gpus} is not supported: this build measures one MI355X "
            "(the attention path shards by batch with no communication; see DESIGN.md)",
            file=sys.stderr,
        )
        return 2
    import torch

    from ataraxos_amd import _lib, ops

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    _lib.load()
    dev = torch.device("cuda:0")
    if args.mode == "pmc":
        pmc_workload(torch, ops, args.batch, args.steps, dev, args.pmc_kernel)
        return 0
    batch, seq, embed, heads, head_dim = args.batch, 100, 384, 6, 64
    t0 = time.time()
    layers = make_layers(torch, batch, seq, embed, args.layers, dev, packed=args.qkv == "packed")
    torch.cuda.synchronize()
    print(f"[bench] inputs ready in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)

    ms_step, kern_mean_ms, kern_ms, kern_min_ms = time_attention(
        torch, ops, layers, heads, head_dim, args.steps, args.warmup)
    del layers
    print(f"[bench] attention timed: {ms_step:.3f} ms/step, {kern_ms * 1e3:.1f} us/launch (median)",
          file=sys.stderr, flush=True)

    bytes_per_sample = 4 * seq * embed * 2  # Q, K, V read + O written, bf16
    flops_per_sample = 4 * heads * seq * seq * head_dim
    value = args.layers * batch / (ms_step * 1e-3)
    # roofline from the median launch (BASELINE's GPU method: median of >= 50)
    achieved = batch * bytes_per_sample / (kern_ms * 1e-3) / 1e9
    tflops = batch * flops_per_sample / (kern_ms * 1e-3) / 1e12
    traffic = None
    if TRAFFIC_FILE.exists():
        try:
            tr = json.loads(TRAFFIC_FILE.read_text())
            if tr.get("batch") == batch:
                traffic = tr.get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None

    result = {
        "metric": METRIC,
        "value": value,
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) tokens through random-init N(0,0.02) QKV projections, resident in HBM",
        "config": {
            "workload": "C3 Move-net encoder self-attention core, 8 layers (value = samples/s per layer)",
            "batch": batch,
            "seq_len": seq,
            "embed_dim": embed,
            "heads": heads,
            "head_dim": head_dim,
            "layers": args.layers,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "kernel": "attn_fwd_16bit<bf16, D=64, NKC=4>",
            "kernel_us_median": kern_ms * 1e3,
            "kernel_us_mean": kern_mean_ms * 1e3,
            "kernel_us_min": kern_min_ms * 1e3,
            "launches_timed": args.steps * args.layers,
            "algorithmic_bytes_per_launch": batch * bytes_per_sample,
        },
        "mfma": {
            "achieved_tflops": tflops,
            "peak_tflops": BF16_PEAK_TFLOPS,
            "frac": tflops / BF16_PEAK_TFLOPS,
            "algorithmic_flops_per_launch": batch * flops_per_sample,
        },
    }
    if not args.no_extras:
        e2e_ms = time_e2e(torch, batch, seq, embed, heads, args.layers, max(5, args.steps // 5), 3, dev, fuse=True)
        unf_ms = time_e2e(torch, batch, seq, embed, heads, args.layers, max(5, args.steps // 5), 3, dev, fuse=False)
        layer_flops = batch * (4 * 2 * seq * embed * embed + heads * 2 * 2 * seq * seq * (embed // heads))
        result["e2e"] = {
            "what": "MultiHeadAttention forward x8 + residual as the module runs it in inference: per layer one launch rearranging the four weights into the fused kernel's tile order, one launch of the fused layer",
            "ms_per_step": e2e_ms,
            "samples_per_s": batch / (e2e_ms * 1e-3),
            "mfma_tflops": args.layers * layer_flops / (e2e_ms * 1e-3) / 1e12,
            "mfma_frac": args.layers * layer_flops / (e2e_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
            "unfused_ms_per_step": unf_ms,
            "unfused_what": "QKV + out projections on hipBLASLt, the attention kernel, residual",
        }
        # One C3 layer through the fused kernel alone (packed weights), per launch.
        gw = torch.Generator(device=dev).manual_seed(46)
        xw = torch.randn(batch, seq, embed, generator=gw, device=dev).to(torch.bfloat16)
        wl = [ops.mha_pack_weight((torch.randn(embed, embed, generator=gw, device=dev) * 0.02).to(torch.bfloat16)) for _ in range(4)]
        yl = torch.empty_like(xw)
        layer_ms = _mean_launch_ms(
            torch, lambda: ops.mha_forward(xw, *wl, num_heads=heads, out=yl, packed=True), args.steps, args.warmup
        )
        result["e2e"]["fused_layer"] = {
            "what": "one C3 layer (B=4096, L=100, 6x64) through atx_mha_fwd_packed: q/k/v projections, attention, output projection",
            "kernel_us": layer_ms * 1e3,
            "samples_per_s": batch / (layer_ms * 1e-3),
            "mfma_tflops": layer_flops / (layer_ms * 1e-3) / 1e12,
            "mfma_frac": layer_flops / (layer_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
        }
        reps = max(5, args.steps // 5)
        chain_ms = time_chain(torch, ops, batch, seq, embed, heads, args.layers, reps, 3, dev)
        result["e2e"]["residual_in_kernel"] = {
            "what": "the same 8-layer chain x <- x + MHA(x) with the residual added inside the fused layer "
                    "(per layer: one weight-rearranging launch, one launch of atx_mha_fwd_ws with residual=1)",
            "ms_per_step": chain_ms,
            "samples_per_s": batch / (chain_ms * 1e-3),
            "mfma_frac": args.layers * layer_flops / (chain_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
            "per_layer_us": chain_ms * 1e3 / args.layers,
        }
        pre_ms = time_chain(torch, ops, batch, seq, embed, heads, args.layers, reps, 3, dev, ln=True)
        pre_unf_ms = time_chain(torch, ops, batch, seq, embed, heads, args.layers, reps, 3, dev, ln=True, fuse=False)
        result["e2e"]["preln_block_half"] = {
            "what": "8 pre-LN block attention halves x <- x + MHA(LayerNorm(x)) (transformer.py:143), each one "
                    "launch (LayerNorm, projections, attention, output projection, residual) after the weight "
                    "rearrangement; unfused: torch LayerNorm, the fused layer, a separate add",
            "ms_per_step": pre_ms,
            "per_layer_us": pre_ms * 1e3 / args.layers,
            "mfma_frac": args.layers * layer_flops / (pre_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
            "unfused_ms_per_step": pre_unf_ms,
        }
        # The reference Move network's own layer: 8 heads x 48 at 101 positions.
        gm = torch.Generator(device=dev).manual_seed(48)
        xm = torch.randn(batch, 101, embed, generator=gm, device=dev).to(torch.bfloat16)
        wm = [ops.mha_pack_weight((torch.randn(embed, embed, generator=gm, device=dev) * 0.02).to(torch.bfloat16)) for _ in range(4)]
        ym = torch.empty_like(xm)
        move_ms = _mean_launch_ms(torch, lambda: ops.mha_forward(xm, *wm, num_heads=8, out=ym, packed=True), args.steps, args.warmup)
        move_flops = batch * (4 * 2 * 101 * embed * embed + 8 * 2 * 2 * 101 * 101 * 48)
        result["e2e"]["fused_layer_move_ref_8x48"] = {
            "what": "one layer of the reference Move network's own shape (B=4096, L=101, 8 heads x 48) "
                    "through atx_mha_fwd_packed",
            "kernel_us": move_ms * 1e3,
            "samples_per_s": batch / (move_ms * 1e-3),
            "mfma_frac": move_flops / (move_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
        }
        result["kq_policy"] = time_kq(torch, ops, batch, dev, args.steps, args.warmup)
        result["belief_attention"] = time_belief(torch, ops, dev, args.steps, args.warmup)
        result["decode"] = time_decode(torch, ops, dev, max(3, args.steps // 10))
        result["backward"] = time_backward(torch, ops, batch, dev, args.steps, args.warmup)
        result["kq_backward"] = time_kq_backward(torch, ops, batch, dev, args.steps, args.warmup)
        result["rollout"] = time_rollout(torch, dev, args.steps, args.warmup)
        print("[bench] extras timed", file=sys.stderr, flush=True)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.cpu_sample)
        print("[bench] cpu baseline timed", file=sys.stderr, flush=True)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
