"""The PPO-update workloads this package is measured on (shapes, synthetic-rollout statistics, hyperparameters).

humanoid (the headline): actor obs 96 -> [512, 256, 128] ELU -> 29 actions, critic obs 99 -> [512, 256, 128] ELU
-> 1, per-dimension observation normalisation, 4096 envs x 24 steps, 5 epochs x 4 mini-batches, gamma 0.99,
lambda 0.95, clip 0.2, clipped value loss, value coef 1.0, entropy coef 0.01, Adam lr 1e-3 with the adaptive-KL
schedule (desired KL 0.01), max grad norm 1.0.  The others vary observation width, env count or the model.
"""

from __future__ import annotations

import copy

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

ALGORITHM = dict(num_learning_epochs=5, num_mini_batches=4, clip_param=0.2, gamma=0.99, lam=0.95,
                 value_loss_coef=1.0, entropy_coef=0.01, learning_rate=1e-3, max_grad_norm=1.0,
                 use_clipped_value_loss=True, schedule="adaptive", desired_kl=0.01)


def train_cfg(workload: dict, algorithm_class: str = "tt_rsl_rl_amd.ppo:PPO", **alg_overrides) -> dict:
    """Runner-style config (upstream layout: algorithm / actor / critic / obs_groups / num_steps_per_env)."""
    model = "RNNModel" if "rnn" in workload else "MLPModel"
    actor = dict(class_name=model, hidden_dims=list(workload["hidden_dims"]), activation="elu",
                 obs_normalization=workload["obs_normalization"],
                 distribution_cfg=dict(class_name="GaussianDistribution", init_std=1.0, std_type="log"))
    critic = dict(class_name=model, hidden_dims=list(workload["hidden_dims"]), activation="elu",
                  obs_normalization=workload["obs_normalization"])
    if "rnn" in workload:
        actor.update(workload["rnn"])
        critic.update(workload["rnn"])
    alg = dict(ALGORITHM, class_name=algorithm_class)
    alg.update(alg_overrides)
    return dict(algorithm=alg, actor=actor, critic=critic, obs_groups=copy.deepcopy(workload["obs_groups"]),
                num_steps_per_env=workload["steps"])


def linear_shapes(workload: dict) -> list[list[tuple[int, int]]]:
    """(in, out) of every linear layer of the actor and of the critic."""
    dims = workload["obs"]
    groups = workload["obs_groups"]
    out = []
    for model, od in (("actor", workload["num_actions"]), ("critic", 1)):
        d_in = sum(dims[g][1] for g in groups[model])
        if "rnn" in workload:  # the head reads the LSTM output
            d_in = workload["rnn"]["rnn_hidden_dim"]
        hs = list(workload["hidden_dims"])
        chain = [d_in] + hs + [od]
        out.append(list(zip(chain[:-1], chain[1:])))
    return out


def gemm_flops_per_update(workload: dict, epochs: int = 5) -> float:
    """Algorithmic GEMM FLOPs of one update: per sample-visit 2*in*out for each of forward, input-grad and
    weight-grad of every layer, except no input-grad for the first layer; B * epochs sample-visits."""
    B = workload["num_envs"] * workload["steps"]
    if "rnn" in workload:
        return lstm_gemm_flops_per_update(workload, epochs)
    per = 0
    for layers in linear_shapes(workload):
        per += sum(3 * 2 * i * o for i, o in layers) - 2 * layers[0][0] * layers[0][1]
    return float(per) * B * epochs


def lstm_gemm_flops_per_update(workload: dict, epochs: int = 5) -> float:
    """Recurrent models (LSTM layers of hidden H, the first on D observation columns and each later one on the h of
    the layer below, then the MLP head), per model, layer and sample-visit: LSTM forward 2*4H*(D_k+H) (input
    projection + recurrent product), weight-grad 2*4H*(D_k+H), the recurrent input-grad 2*4H*H on all but the last
    step of each sequence (no gradient flows into the saved initial state), for a layer above the first the
    input-grad 2*4H*H into the lower layer's outputs (none into the observations); the head: forward, input-grad and
    weight-grad of every layer (its first layer's input-grad feeds the top LSTM layer)."""
    N, T = workload["num_envs"], workload["steps"]
    B = N * T
    H = workload["rnn"]["rnn_hidden_dim"]
    layers_rnn = workload["rnn"].get("rnn_num_layers", 1)
    dims, groups = workload["obs"], workload["obs_groups"]
    total = 0
    for layers, model in zip(linear_shapes(workload), ("actor", "critic")):
        D = sum(dims[g][1] for g in groups[model])
        total += B * sum(3 * 2 * i * o for i, o in layers)
        for k in range(layers_rnn):
            Dk = D if k == 0 else H
            total += B * 2 * 2 * 4 * H * (Dk + H) + (B - N) * 2 * 4 * H * H
            if k > 0:
                total += B * 2 * 4 * H * H
    return float(total) * epochs
