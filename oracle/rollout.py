"""Synthetic rollouts for the PPO update workloads (test infrastructure only; see ``oracle/__init__.py``).

A rollout is generated ONCE on the CPU by the oracle (the upstream restatement), as the reference's own
benchmark does with a null environment (scripts/bench_matrix.py:34-51): seeded observations, actions sampled
from the policy, rewards ~ N(0, s^2), Bernoulli dones, bootstrap values from the critic.  The same record is
then handed to the oracle and to the device implementation through ``add_transition``.
"""

from __future__ import annotations

import copy
from dataclasses import dataclass, field

import torch

from .ppo_ref import PPO, Transition, construct_algorithm

# Workload table.  obs: group -> (distribution, width); groups are concatenated in the listed order.
WORKLOADS: dict[str, dict] = {
    "flat48": dict(num_envs=4096, steps=24, obs={"policy": ("normal", 48)},
                   obs_groups={"actor": ["policy"], "critic": ["policy"]}, num_actions=12,
                   hidden_dims=[512, 256, 128], reward_std=0.1, p_done=0.005, obs_normalization=False),
    "humanoid": dict(num_envs=4096, steps=24, obs={"policy": ("normal", 96), "critic": ("normal", 99)},
                     obs_groups={"actor": ["policy"], "critic": ["critic"]}, num_actions=29,
                     hidden_dims=[512, 256, 128], reward_std=0.2, p_done=0.01, obs_normalization=True),
    "rough235": dict(num_envs=4096, steps=24, obs={"policy": ("normal", 48), "height_scan": ("uniform", 187)},
                     obs_groups={"actor": ["policy", "height_scan"], "critic": ["policy", "height_scan"]},
                     num_actions=12, hidden_dims=[512, 256, 128], reward_std=0.1, p_done=0.005,
                     obs_normalization=False),
    "flat48_65k": dict(num_envs=65536, steps=24, obs={"policy": ("normal", 48)},
                       obs_groups={"actor": ["policy"], "critic": ["policy"]}, num_actions=12,
                       hidden_dims=[512, 256, 128], reward_std=0.1, p_done=0.005, obs_normalization=False),
    "lstm256": dict(num_envs=4096, steps=24, obs={"policy": ("normal", 48)},
                    obs_groups={"actor": ["policy"], "critic": ["policy"]}, num_actions=12,
                    hidden_dims=[256, 128], reward_std=0.1, p_done=0.01, obs_normalization=False,
                    rnn=dict(rnn_type="lstm", rnn_hidden_dim=256, rnn_num_layers=1)),
}

DEFAULT_ALGORITHM = dict(num_learning_epochs=5, num_mini_batches=4, clip_param=0.2, gamma=0.99, lam=0.95,
                         value_loss_coef=1.0, entropy_coef=0.01, learning_rate=1e-3, max_grad_norm=1.0,
                         use_clipped_value_loss=True, schedule="adaptive", desired_kl=0.01)


def train_cfg(workload: dict, algorithm_class: str = "PPO", **alg_overrides) -> dict:
    """The runner-style config of a workload (upstream layout: algorithm / actor / critic / obs_groups)."""
    model = "RNNModel" if "rnn" in workload else "MLPModel"
    actor = dict(class_name=model, hidden_dims=list(workload["hidden_dims"]), activation=workload.get("activation", "elu"),
                 obs_normalization=workload["obs_normalization"],
                 distribution_cfg=dict(class_name="GaussianDistribution", init_std=1.0, std_type="log"))
    if workload.get("learn_std") is False:  # a fixed std (distribution.py:166)
        actor["distribution_cfg"]["learn_std"] = False
    critic = dict(class_name=model, hidden_dims=list(workload["hidden_dims"]),
                  activation=workload.get("critic_activation", workload.get("activation", "elu")),
                  obs_normalization=workload["obs_normalization"])
    if "rnn" in workload:
        actor.update(workload["rnn"])
        critic.update(workload["rnn"])
    alg = dict(DEFAULT_ALGORITHM, class_name=algorithm_class)
    alg.update(alg_overrides)
    return dict(algorithm=alg, actor=actor, critic=critic, obs_groups=copy.deepcopy(workload["obs_groups"]),
                num_steps_per_env=workload["steps"])


def scaled(workload: dict, num_envs: int | None = None, steps: int | None = None, hidden_dims=None) -> dict:
    w = copy.deepcopy(workload)
    if num_envs is not None:
        w["num_envs"] = num_envs
    if steps is not None:
        w["steps"] = steps
    if hidden_dims is not None:
        w["hidden_dims"] = list(hidden_dims)
    return w


def sample_obs(workload: dict, n: int | None = None) -> dict:
    n = workload["num_envs"] if n is None else n
    out = {}
    for name, (kind, width) in workload["obs"].items():
        if kind == "normal":
            out[name] = torch.randn(n, width)
        else:
            out[name] = torch.rand(n, width) * 2.0 - 1.0
    return out


def zero_obs(workload: dict) -> dict:
    return {name: torch.zeros(workload["num_envs"], w) for name, (_, w) in workload["obs"].items()}


@dataclass
class Rollout:
    """Everything a storage receives during one rollout, step by step (``transitions``), plus the final obs."""

    transitions: list = field(default_factory=list)
    last_obs: dict = field(default_factory=dict)
    init_state: dict = field(default_factory=dict)  # oracle actor/critic state_dicts before the rollout


def make_oracle(workload: dict, seed: int = 0, **alg_overrides) -> PPO:
    torch.manual_seed(seed)
    cfg = train_cfg(workload, **alg_overrides)
    return construct_algorithm(zero_obs(workload), workload["num_envs"], workload["num_actions"], cfg)


def generate(workload: dict, seed: int = 0, carry_state: bool = False, **alg_overrides) -> tuple[PPO, Rollout]:
    """Build the oracle algorithm with ``seed`` and fill its storage with one synthetic rollout.  With
    ``carry_state`` recurrent models start the rollout from a random hidden state (as a rollout after the first
    does), instead of nn.LSTM's zero default."""
    alg = make_oracle(workload, seed, **alg_overrides)
    alg.train_mode()
    roll = Rollout(init_state={"actor": copy.deepcopy(alg.actor.state_dict()),
                               "critic": copy.deepcopy(alg.critic.state_dict())})
    n = workload["num_envs"]
    if carry_state and "rnn" in workload:
        H, layers = workload["rnn"]["rnn_hidden_dim"], workload["rnn"].get("rnn_num_layers", 1)
        gru = workload["rnn"].get("rnn_type", "lstm").lower() == "gru"
        for model in (alg.actor, alg.critic):
            state = tuple(0.5 * torch.randn(layers, n, H) for _ in range(1 if gru else 2))
            model.reset(hidden_state=state[0] if gru else state)
    with torch.inference_mode():
        obs = sample_obs(workload)
        for _ in range(workload["steps"]):
            alg.act(obs)
            tr = alg.transition
            rec = Transition()
            rec.observations = {k: v.clone() for k, v in obs.items()}
            rec.actions = tr.actions.clone()
            rec.values = tr.values.clone()
            rec.actions_log_prob = tr.actions_log_prob.clone()
            rec.distribution_params = tuple(p.clone() for p in tr.distribution_params)
            hs = tr.hidden_states
            rec.hidden_states = tuple(None if h is None else (tuple(x.clone() for x in h) if isinstance(h, tuple)
                                                               else h.clone()) for h in hs)
            rewards = workload["reward_std"] * torch.randn(n)
            dones = (torch.rand(n) < workload["p_done"]).float()
            rec.rewards = rewards.clone()
            rec.dones = dones.clone()
            roll.transitions.append(rec)
            obs = sample_obs(workload)
            alg.process_env_step(obs, rewards, dones, {})
        roll.last_obs = {k: v.clone() for k, v in obs.items()}
    return alg, roll


def feed(storage, roll: Rollout) -> None:
    """Replay a recorded rollout into any storage exposing upstream's ``add_transition`` / ``clear``."""
    storage.clear()
    for rec in roll.transitions:
        storage.add_transition(rec)
