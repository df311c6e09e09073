"""qqtsim: the self-play rollout hot path of the bomber simulator on MI355X.

`HipBatchedSim` (the reference's `BatchedSim` API), `HipActorCritic` (the mlp
`ActorCritic.act/forward/evaluate` API; `HipCnnActorCritic`,
`HipLstmActorCritic` for the cnn and lstm archs), `Rollout` (observe -> act ->
step in two launches; `LstmRollout` for the lstm arch), `HipRolloutBuffer` / `compute_gae`, `HipMlpActorCritic` /
`ppo_update` (the PPO update with the first layer's forward and weight
gradient on MFMA) and `make_sim`, all over hand-written HIP kernels in
libqqt_hip.so (C ABI in include/qqt_hip.h).  Importing the package does not
load the library; the first sim or policy does, and raises if it is missing.
"""

from .bots import HipAstarBot
from .learn import HipMlpActorCritic, LstmLearner, PPOConfig, ppo_update
from .config import SimConfig, corridor_training_config
from .factory import make_sim
from .maps import BOMB_STRESS_40, CORRIDOR_70, OPEN_PILLARS, MapSpec
from .policy import (HipActorCritic, HipCnnActorCritic, HipLstmActorCritic, default_init,
                     default_init_cnn, reference_init)
from .ppo import HipRolloutBuffer, compute_gae
from .rollout import LstmRollout, Rollout
from .sim import HipBatchedSim

__all__ = ["HipAstarBot", "SimConfig", "corridor_training_config", "make_sim", "MapSpec",
           "OPEN_PILLARS", "CORRIDOR_70", "BOMB_STRESS_40", "HipActorCritic", "HipCnnActorCritic",
           "HipLstmActorCritic", "default_init", "default_init_cnn", "reference_init", "Rollout",
           "LstmRollout", "HipBatchedSim", "HipRolloutBuffer", "compute_gae",
           "HipMlpActorCritic", "LstmLearner", "PPOConfig", "ppo_update"]
