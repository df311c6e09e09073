"""`qqtsim.policy.reference_init` against the weights the reference's own
`ActorCritic` holds after `torch.manual_seed(0)` (train/model.py:154-165),
as `tests/golden/gen_reference_vectors.py` wrote them into `mlp.npz`,
`cnn.npz` and `lstm.npz`.

The generator perturbed every bias, the LayerNorm affines and (cnn) every
`conv.*` parameter by `0.1 * randn` from `Generator().manual_seed(1)`,
drawn in `named_parameters()` order, before saving (lstm: only the biases,
from `Generator().manual_seed(2)`).  The unperturbed
parameters (the Linear / conv0 weights: orthogonal draws) are compared bit
for bit; the perturbed ones must equal the init plus the replayed
perturbation, which pins zero biases and LayerNorm 1 / 0.  Planted
mistakes (gain 1 instead of sqrt 2, no second draw for the policy heads'
output layers, the heads' layers drawn before the trunk) must fail."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from qqtsim.policy import _layer_tree, _tree_state, default_init, reference_init

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _perturbed(name: str, arch: str) -> bool:
    if arch == "lstm":
        return "bias" in name
    return (name.endswith("bias") or ".1." in name or ".4." in name
            or (arch == "cnn" and name.startswith("conv.")))


def _golden(arch: str) -> dict:
    z = np.load(os.path.join(GOLDEN, f"{arch}.npz"))
    return {k[2:]: z[k] for k in z.files if k.startswith("w_")}


def _mismatches(sd: dict, arch: str) -> list[str]:
    """Names of parameters where `sd` (as the reference init) and the golden
    weights disagree once the generator's perturbation is replayed."""
    gold = _golden(arch)
    g = torch.Generator().manual_seed(2 if arch == "lstm" else 1)
    bad = []
    names = [n for n, _ in _layer_tree(arch, (14, 13, 13), 5, 2).named_parameters()]
    for name in names:
        key = name.replace(".", "_")
        want = torch.from_numpy(gold[key])
        got = sd[name].clone()
        if _perturbed(name, arch):
            got = got.add_(0.1 * torch.randn(got.shape, generator=g))
        if got.shape != want.shape or not torch.equal(got, want):
            bad.append(name)
    return bad


@pytest.mark.parametrize("arch", ["mlp", "cnn", "lstm"])
def test_reference_init_equals_reference_weights(arch):
    """lstm: the torch.nn.LSTM's own uniform init, drawn when the layer is
    built between l_fusion and the heads, is part of what is pinned."""
    sd = reference_init(seed=0, arch=arch)
    gold = _golden(arch)
    assert set(k.replace(".", "_") for k in sd) == set(gold), "state_dict keys differ"
    assert _mismatches(sd, arch) == []
    n = sum(v.numel() for v in sd.values())
    assert n == {"mlp": 345_288, "cnn": 281_744, "lstm": 368_816}[arch]


def test_reference_init_structure():
    """Orthogonality and gains of what reference_init draws: W W^T = 2 I for
    the gain-sqrt(2) layers (rows <= cols), W^T W = 2 I otherwise, 1e-4 I
    for the two policy output layers, zero biases, LayerNorm 1 / 0."""
    sd = reference_init(seed=3)
    for k, w in sd.items():
        if k.endswith("weight") and w.dim() == 2:
            gain2 = 1e-4 if k in ("move_head.2.weight", "bomb_head.2.weight") else 2.0
            m = w @ w.t() if w.shape[0] <= w.shape[1] else w.t() @ w
            eye = torch.eye(m.shape[0]) * gain2
            assert torch.allclose(m, eye, atol=1e-5 * gain2 * 10), k
        elif k.endswith("bias"):
            assert torch.count_nonzero(w) == 0, k
        else:
            assert torch.equal(w, torch.ones_like(w)), k


def _planted(kind: str) -> dict:
    nn = torch.nn
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(0)
        tree = _layer_tree("mlp", (14, 13, 13), 5, 2)
        mods = [m for m in tree.modules() if isinstance(m, nn.Linear)]
        if kind == "heads_first":
            mods = mods[2:] + mods[:2]
        with torch.no_grad():
            for m in mods:
                nn.init.orthogonal_(m.weight, gain=1.0 if kind == "gain1" else 2 ** 0.5)
                nn.init.zeros_(m.bias)
            if kind != "no_head_redraw":
                for head in (tree.move_head, tree.bomb_head):
                    nn.init.orthogonal_(head[-1].weight, gain=0.01)
        return _tree_state(tree)


@pytest.mark.parametrize("kind", ["gain1", "no_head_redraw", "heads_first"])
def test_planted_init_mistakes_fail(kind):
    assert _mismatches(_planted(kind), "mlp") != []


def test_default_init_is_not_the_reference_init():
    """PyTorch's default Linear init (the benchmark workload's weights) is a
    different distribution: it must not pass as the reference init."""
    assert _mismatches(default_init(), "mlp") != []
