"""CPU oracle for the attention hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or, for the
baseline, as the thing timed on the host CPU).  The product package
``ataraxos_amd`` never imports it; its GPU path fails loudly instead of
falling back to anything here.

Modules (each function cites the reference file:line it restates):

* :mod:`oracle.attention` — numpy float64 restatement of
  ``MultiHeadAttention._forward_math`` (stratego/networks/attention.py:281-316),
  the GQA expansion (:210-220) and the module forward (:152-204), and the
  gradients autograd takes through that math (stratego/training/move_trainer.py:140).
* :mod:`oracle.policy` — the key-query policy head's logits and mask
  (stratego/networks/move_net.py:89-95) and the callers' softmax
  (stratego/training/selfplay.py:284).
* :mod:`oracle.decode` — one incremental-decode step as the last row of the
  full causal recompute the reference performs (selfplay.py:139-146,181).
* :mod:`oracle.cpu_baseline` — a torch-on-CPU port of the same math path,
  timed as the reported CPU baseline.
* :mod:`oracle.rollout` (+ ``rollout.c``, built with gcc) — the self-play
  simulator of csrc/stratego_buffer.cu / .cpp: apply_actions, the legal-move
  mask, reset, the infostate and the Zobrist hash, one loop per game.  Pinned
  by the reference's own simulator tests, whose positions and expected
  values are known answers (tests/_rollout_scenarios.py), and by two code
  paths that must agree: the mask against apply's validation over all 10,000
  actions, the mask's "any move" against the no-move loss; the hash by its
  XOR-linearity.

Pinning.  The reference holds no golden values for this path (its tests check
invariants only), so every oracle function is pinned by checks in
``tests/test_oracle_*.py`` against results it does not share code with:
torch's ``scaled_dot_product_attention`` and ``nn.MultiheadAttention`` on the
CPU in float64 (and torch autograd through them for the gradients), central
finite differences of the forward, scipy's ``softmax``, closed forms (one key, constant keys,
one dominant logit, causal row 0, a single legal move, equal logits), the
reference's own invariants, and planted-mistake tests showing that each
check rejects a wrong variant.  No function here is "parity unpinned".
"""
