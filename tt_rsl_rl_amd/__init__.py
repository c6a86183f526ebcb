"""MI355X-native (gfx950) PPO update path for rsl_rl, as a plugin: ``"tt_rsl_rl_amd.ppo:PPO"``.

Host code mirrors upstream rsl_rl's PPO / RolloutStorage / MLPModel interface; the arithmetic runs in the HIP
kernels of ``libppo_hip.so`` (C ABI: ``include/ppo_hip.h``), loaded through ctypes.
"""

from .models import EmpiricalNormalization, GaussianDistribution, MLPModel
from .ppo import PPO, HipPPO
from .storage import RolloutStorage

__all__ = ["PPO", "HipPPO", "MLPModel", "GaussianDistribution", "EmpiricalNormalization", "RolloutStorage"]
