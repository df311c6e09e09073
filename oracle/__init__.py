"""CPU oracle for the rollout hot path.  TEST INFRASTRUCTURE ONLY.

This package restates, in plain PyTorch tensor ops, the reference's rollout
tick (sim/torch_sim.py `BatchedSim.step/observe/legal_mask`, sim/blast.py,
sim/move.py, sim/obs.py) and the MLP actor/critic forward + masked sampling
(train/model.py).  It exists to check the HIP path and to serve as the
timed CPU baseline; it is never the product.  Only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
it.  The HIP path never falls back to it.

Each function cites the reference file:line it follows.  What pins each
function (reference golden vectors, closed-form rule tests, textbook
identities) is listed in the test modules under `tests/` that exercise it;
the randomness helpers (`philox`, `maps`) define the injected-randomness
convention shared with the HIP path and are pinned by the Philox known-answer
vectors of the Random123 paper.
"""
