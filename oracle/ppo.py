"""CPU restatement of the reference's advantage estimation (test
infrastructure only: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg).

`gae` follows compute_gae (train/ppo.py:101-110) step for step in float32
with the reference's operation order.  The reference multiplies float32
tensors by Python floats, which torch applies as float32(scalar) (checked
against torch in tests/test_oracle_ppo.py), and forms `gamma * lam` as a
double product before it meets a tensor.  Pinned by closed forms (lam = 0,
all-terminal, undiscounted sums), a float64 recurrence within float32
tolerance, and torch's own evaluation of the reference expression.
"""

from __future__ import annotations

import numpy as np


def gae(rew, val, done, last_val, gamma: float, lam: float):
    """(adv, ret) float32 (T, N) from rew/val/done (T, N) and last_val (N,)
    (train/ppo.py:101-110)."""
    rew = np.asarray(rew, dtype=np.float32)
    val = np.asarray(val, dtype=np.float32)
    done = np.asarray(done, dtype=np.float32)
    last_val = np.asarray(last_val, dtype=np.float32)
    g = np.float32(gamma)
    gl = np.float32(gamma * lam)            # Python evaluates gamma * lam first, in double
    steps = rew.shape[0]
    adv = np.zeros_like(rew)
    run = np.zeros_like(last_val)
    for t in reversed(range(steps)):
        nonterminal = np.float32(1.0) - done[t]
        next_val = last_val if t == steps - 1 else val[t + 1]
        delta = (rew[t] + (g * next_val) * nonterminal) - val[t]
        run = delta + (gl * nonterminal) * run
        adv[t] = run
    return adv, adv + val
