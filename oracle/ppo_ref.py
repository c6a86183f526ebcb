"""CPU restatement of upstream rsl_rl v5.5.2 PPO (test infrastructure only; see ``oracle/__init__.py``).

Every class and function names the upstream file:line it restates.  Observations are plain
``dict[str, Tensor]`` (upstream uses ``tensordict.TensorDict``, which only acts as a container on this path).
"""

from __future__ import annotations

import math
import warnings
from itertools import chain
from typing import Callable, Mapping

import numpy as np
import torch
import torch.nn as nn
from torch.distributions import Normal

ObsDict = dict


# ----------------------------------------------------------------------------------------------------------------------
# utils (rsl_rl/utils/utils.py)
# ----------------------------------------------------------------------------------------------------------------------


def activation_module(name: str) -> nn.Module:
    """rsl_rl/utils/utils.py:34-68 -- one module instance, shared by every hidden layer of an MLP."""
    table: dict[str, Callable[[], nn.Module]] = {
        "elu": nn.ELU,
        "selu": nn.SELU,
        "relu": nn.ReLU,
        "crelu": nn.CELU,
        "lrelu": nn.LeakyReLU,
        "tanh": nn.Tanh,
        "sigmoid": nn.Sigmoid,
        "softplus": nn.Softplus,
        "gelu": nn.GELU,
        "swish": nn.SiLU,
        "mish": nn.Mish,
        "identity": nn.Identity,
    }
    key = name.lower()
    if key not in table:
        raise ValueError(f"Invalid activation function '{name}'. Valid activations are: {list(table)}")
    return table[key]()


def resolve_obs_groups(obs: Mapping, obs_groups: dict, default_sets: list[str]) -> dict:
    """rsl_rl/utils/utils.py:192-287 (the printing is dropped)."""
    if len(obs_groups) == 0:
        warnings.warn("The observation configuration dictionary 'obs_groups' is empty.")
    else:
        for set_name, groups in obs_groups.items():
            if len(groups) == 0:
                raise ValueError(f"The '{set_name}' key in the 'obs_groups' dictionary can not be an empty list.")
            for group in groups:
                if group not in obs:
                    raise ValueError(f"Observation '{group}' in observation set '{set_name}' not found.")
    for name in default_sets:
        if name in obs_groups:
            continue
        if name in obs:
            obs_groups[name] = [name]
        elif "policy" in obs:
            obs_groups[name] = ["policy"]
        else:
            raise ValueError(f"The observation configuration dictionary 'obs_groups' does not contain '{name}'.")
    return obs_groups


def split_and_pad_trajectories(tensor, dones: torch.Tensor):
    """rsl_rl/utils/utils.py:395-449 for a tensor or a dict of tensors laid out [T, N, ...]."""
    dones = dones.clone()
    dones[-1] = 1
    flat_dones = dones.transpose(1, 0).reshape(-1, 1)
    done_idx = torch.cat((flat_dones.new_tensor([-1], dtype=torch.int64), flat_dones.nonzero()[:, 0]))
    lengths = done_idx[1:] - done_idx[:-1]
    lengths_list = lengths.tolist()

    def pad_one(v: torch.Tensor) -> torch.Tensor:
        pieces = torch.split(v.transpose(1, 0).flatten(0, 1), lengths_list)
        pieces = (*pieces, torch.zeros(v.shape[0], *v.shape[2:], device=v.device))
        return torch.nn.utils.rnn.pad_sequence(pieces)[:, :-1]

    if isinstance(tensor, Mapping):
        padded = {k: pad_one(v) for k, v in tensor.items()}
        t_len = next(iter(tensor.values())).shape[0]
    else:
        padded = pad_one(tensor)
        t_len = tensor.shape[0]
    masks = lengths > torch.arange(0, t_len, device=dones.device).unsqueeze(1)
    return padded, masks


def unpad_trajectories(trajectories, masks: torch.Tensor):
    """rsl_rl/utils/utils.py:452-463 (tensor form; dicts are unpadded key by key)."""
    if isinstance(trajectories, Mapping):
        return {k: unpad_trajectories(v, masks) for k, v in trajectories.items()}
    valid = trajectories.transpose(1, 0)[masks.transpose(1, 0)]
    return valid.view(-1, trajectories.shape[0], *trajectories.shape[2:]).transpose(1, 0)


# ----------------------------------------------------------------------------------------------------------------------
# modules
# ----------------------------------------------------------------------------------------------------------------------


class EmpiricalNormalization(nn.Module):
    """rsl_rl/modules/normalization.py:15-78 (single process: the all-reduce branch never runs)."""

    def __init__(self, shape, eps: float = 1e-2, until: int | None = None) -> None:
        super().__init__()
        self.eps = eps
        self.until = until
        self.register_buffer("_mean", torch.zeros(shape).unsqueeze(0))
        self.register_buffer("_var", torch.ones(shape).unsqueeze(0))
        self.register_buffer("_std", torch.ones(shape).unsqueeze(0))
        self.register_buffer("count", torch.tensor(0, dtype=torch.long))

    @property
    def mean(self) -> torch.Tensor:
        return self._mean.squeeze(0).clone()

    @property
    def std(self) -> torch.Tensor:
        return self._std.squeeze(0).clone()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return (x - self._mean) / (self._std + self.eps)

    def update(self, x: torch.Tensor) -> None:
        if not self.training:
            return
        if self.until is not None and self.count >= self.until:
            return
        n = torch.tensor(x.shape[0], dtype=self.count.dtype)
        batch_var = torch.var(x, dim=0, unbiased=False, keepdim=True)
        batch_mean = torch.mean(x, dim=0, keepdim=True)
        self.count += n
        rate = n / self.count
        delta = batch_mean - self._mean
        self._mean += rate * delta
        self._var += rate * (batch_var - self._var + delta * (batch_mean - self._mean))
        self._std = torch.sqrt(self._var)


class GaussianDistribution(nn.Module):
    """rsl_rl/modules/distribution.py:132-238 (state-independent std, ``scalar`` or ``log`` parameterisation)."""

    def __init__(self, output_dim: int, init_std: float = 1.0, std_range=(1e-6, 1e6), std_type: str = "scalar",
                 learn_std: bool = True) -> None:
        super().__init__()
        self.output_dim = output_dim
        self.std_type = std_type
        if std_type == "scalar":
            self.std_param = nn.Parameter(init_std * torch.ones(output_dim), requires_grad=learn_std)
        elif std_type == "log":
            self.log_std_param = nn.Parameter(torch.log(init_std * torch.ones(output_dim)), requires_grad=learn_std)
        else:
            raise ValueError(f"Unknown standard deviation type: {std_type}. Should be 'scalar' or 'log'.")
        self.std_range = list(std_range)
        self.std_range[0] = max(self.std_range[0], 1e-6)
        self.log_std_range = [float(np.log(self.std_range[0])), float(np.log(self.std_range[1]))]
        self._distribution: Normal | None = None
        Normal.set_default_validate_args(False)

    @property
    def input_dim(self) -> int:
        return self.output_dim

    def current_std(self) -> torch.Tensor:
        if self.std_type == "scalar":
            return self.std_param.clamp(self.std_range[0], self.std_range[1])
        return torch.exp(self.log_std_param.clamp(self.log_std_range[0], self.log_std_range[1]))

    def update(self, mlp_output: torch.Tensor) -> None:
        self._distribution = Normal(mlp_output, self.current_std())

    def sample(self) -> torch.Tensor:
        return self._distribution.sample()

    @property
    def mean(self) -> torch.Tensor:
        return self._distribution.mean

    @property
    def std(self) -> torch.Tensor:
        return self._distribution.stddev

    @property
    def entropy(self) -> torch.Tensor:
        return self._distribution.entropy().sum(dim=-1)

    @property
    def params(self) -> tuple[torch.Tensor, ...]:
        return (self.mean, self.std)

    def log_prob(self, outputs: torch.Tensor) -> torch.Tensor:
        return self._distribution.log_prob(outputs).sum(dim=-1)

    def kl_divergence(self, old_params, new_params) -> torch.Tensor:
        old_mean, old_std = old_params
        new_mean, new_std = new_params
        return torch.distributions.kl_divergence(Normal(old_mean, old_std), Normal(new_mean, new_std)).sum(dim=-1)


class MLP(nn.Sequential):
    """rsl_rl/modules/mlp.py:27-95: Linear, act, ..., Linear (act is ONE shared module instance)."""

    def __init__(self, input_dim: int, output_dim: int, hidden_dims, activation: str = "elu") -> None:
        super().__init__()
        act = activation_module(activation)
        dims = [input_dim if d == -1 else d for d in hidden_dims]
        layers: list[nn.Module] = [nn.Linear(input_dim, dims[0]), act]
        for a, b in zip(dims[:-1], dims[1:]):
            layers += [nn.Linear(a, b), act]
        layers.append(nn.Linear(dims[-1], output_dim))
        for i, layer in enumerate(layers):
            self.add_module(str(i), layer)


class RNN(nn.Module):
    """rsl_rl/modules/rnn.py:22-86 (LSTM / GRU with rollout-mode hidden state, batch-mode unpadding)."""

    def __init__(self, input_size: int, hidden_dim: int = 256, num_layers: int = 1, type: str = "lstm") -> None:
        super().__init__()
        cls = nn.GRU if type.lower() == "gru" else nn.LSTM
        self.rnn = cls(input_size=input_size, hidden_size=hidden_dim, num_layers=num_layers)
        self.hidden_state = None

    def forward(self, x: torch.Tensor, masks=None, hidden_state=None) -> torch.Tensor:
        if masks is not None:
            if hidden_state is None:
                raise ValueError("Hidden states not passed to RNN module during policy update")
            out, _ = self.rnn(x, hidden_state)
            return unpad_trajectories(out, masks)
        out, self.hidden_state = self.rnn(x.unsqueeze(0), self.hidden_state)
        return out

    def reset(self, dones=None, hidden_state=None) -> None:
        if dones is None:
            self.hidden_state = hidden_state
        elif self.hidden_state is not None:
            if hidden_state is not None:
                raise NotImplementedError("custom hidden state on reset")
            states = self.hidden_state if isinstance(self.hidden_state, tuple) else (self.hidden_state,)
            for h in states:
                h[..., dones == 1, :] = 0.0


# ----------------------------------------------------------------------------------------------------------------------
# models
# ----------------------------------------------------------------------------------------------------------------------


class MLPModel(nn.Module):
    """rsl_rl/models/mlp_model.py:30-193.  Registration order (normalizer, distribution, mlp) fixes both the
    state_dict keys and the parameter order (distribution parameter first)."""

    is_recurrent = False

    def __init__(self, obs: Mapping, obs_groups: dict, obs_set: str, output_dim: int, hidden_dims=(256, 256, 256),
                 activation: str = "elu", obs_normalization: bool = False, distribution_cfg: dict | None = None) -> None:
        super().__init__()
        self.obs_groups = list(obs_groups[obs_set])
        self.obs_dim = 0
        for g in self.obs_groups:
            if obs[g].dim() != 2:
                raise ValueError(f"The MLP model only supports 1D observations, got shape {tuple(obs[g].shape)}.")
            self.obs_dim += obs[g].shape[-1]
        self.obs_normalization = obs_normalization
        self.obs_normalizer = EmpiricalNormalization(self.obs_dim) if obs_normalization else nn.Identity()
        if distribution_cfg is not None:
            cfg = dict(distribution_cfg)
            name = cfg.pop("class_name")
            if name.split(":")[-1].split(".")[-1] != "GaussianDistribution":
                raise NotImplementedError(f"distribution {name} is not on the PPO path of this oracle")
            self.distribution: GaussianDistribution | None = GaussianDistribution(output_dim, **cfg)
            mlp_out = self.distribution.input_dim
        else:
            self.distribution = None
            mlp_out = output_dim
        self.mlp = MLP(self._latent_dim(), mlp_out, hidden_dims, activation)

    def _latent_dim(self) -> int:
        return self.obs_dim

    def get_latent(self, obs: Mapping, masks=None, hidden_state=None) -> torch.Tensor:
        return self.obs_normalizer(torch.cat([obs[g] for g in self.obs_groups], dim=-1))

    def forward(self, obs: Mapping, masks=None, hidden_state=None, stochastic_output: bool = False) -> torch.Tensor:
        if masks is not None and not self.is_recurrent:
            obs = unpad_trajectories(obs, masks)
        out = self.mlp(self.get_latent(obs, masks, hidden_state))
        if self.distribution is not None:
            if stochastic_output:
                self.distribution.update(out)
                return self.distribution.sample()
            return out
        return out

    def reset(self, dones=None, hidden_state=None) -> None:
        pass

    def get_hidden_state(self):
        return None

    @property
    def output_mean(self) -> torch.Tensor:
        return self.distribution.mean

    @property
    def output_std(self) -> torch.Tensor:
        return self.distribution.std

    @property
    def output_entropy(self) -> torch.Tensor:
        return self.distribution.entropy

    @property
    def output_distribution_params(self):
        return self.distribution.params

    def get_output_log_prob(self, outputs: torch.Tensor) -> torch.Tensor:
        return self.distribution.log_prob(outputs)

    def get_kl_divergence(self, old_params, new_params) -> torch.Tensor:
        return self.distribution.kl_divergence(old_params, new_params)

    def update_normalization(self, obs: Mapping) -> None:
        if self.obs_normalization and self.obs_groups:
            self.obs_normalizer.update(torch.cat([obs[g] for g in self.obs_groups], dim=-1))


class RNNModel(MLPModel):
    """rsl_rl/models/rnn_model.py:30-96: normalizer -> RNN -> MLP head."""

    is_recurrent = True

    def __init__(self, obs: Mapping, obs_groups: dict, obs_set: str, output_dim: int, hidden_dims=(256, 256, 256),
                 activation: str = "elu", obs_normalization: bool = False, distribution_cfg: dict | None = None,
                 rnn_type: str = "lstm", rnn_hidden_dim: int = 256, rnn_num_layers: int = 1) -> None:
        self.latent_dim = rnn_hidden_dim
        super().__init__(obs, obs_groups, obs_set, output_dim, hidden_dims, activation, obs_normalization,
                         distribution_cfg)
        self.rnn = RNN(self.obs_dim, rnn_hidden_dim, rnn_num_layers, rnn_type)

    def _latent_dim(self) -> int:
        return self.latent_dim

    def get_latent(self, obs: Mapping, masks=None, hidden_state=None) -> torch.Tensor:
        latent = super().get_latent(obs)
        return self.rnn(latent, masks, hidden_state).squeeze(0)

    def reset(self, dones=None, hidden_state=None) -> None:
        self.rnn.reset(dones, hidden_state)

    def get_hidden_state(self):
        return self.rnn.hidden_state


# ----------------------------------------------------------------------------------------------------------------------
# storage (rsl_rl/storage/rollout_storage.py)
# ----------------------------------------------------------------------------------------------------------------------


class Transition:
    """rollout_storage.py:24-65."""

    def __init__(self) -> None:
        self.observations = None
        self.actions = None
        self.rewards = None
        self.dones = None
        self.values = None
        self.actions_log_prob = None
        self.distribution_params = None
        self.hidden_states = (None, None)

    def clear(self) -> None:
        self.__init__()


class Batch:
    """rollout_storage.py:67-123 (RL fields)."""

    def __init__(self, observations=None, actions=None, values=None, advantages=None, returns=None,
                 old_actions_log_prob=None, old_distribution_params=None, hidden_states=(None, None), masks=None,
                 indices=None) -> None:
        self.observations = observations
        self.actions = actions
        self.values = values
        self.advantages = advantages
        self.returns = returns
        self.old_actions_log_prob = old_actions_log_prob
        self.old_distribution_params = old_distribution_params
        self.hidden_states = hidden_states
        self.masks = masks
        self.indices = indices  # the flat row indices of this mini-batch (diagnostic, not upstream)


class RolloutStorage:
    """rollout_storage.py:125-359, ``training_type == "rl"``."""

    def __init__(self, num_envs: int, num_transitions_per_env: int, obs: Mapping, actions_shape) -> None:
        T, N = num_transitions_per_env, num_envs
        self.num_envs = N
        self.num_transitions_per_env = T
        self.actions_shape = list(actions_shape)
        self.observations = {k: torch.zeros(T, *v.shape, dtype=v.dtype) for k, v in obs.items()}
        self.rewards = torch.zeros(T, N, 1)
        self.actions = torch.zeros(T, N, *actions_shape)
        self.dones = torch.zeros(T, N, 1).byte()
        self.values = torch.zeros(T, N, 1)
        self.actions_log_prob = torch.zeros(T, N, 1)
        self.distribution_params: tuple[torch.Tensor, ...] | None = None
        self.returns = torch.zeros(T, N, 1)
        self.advantages = torch.zeros(T, N, 1)
        self.saved_hidden_state_a = None
        self.saved_hidden_state_c = None
        self.step = 0

    def add_transition(self, t: Transition) -> None:
        """rollout_storage.py:173-205."""
        if self.step >= self.num_transitions_per_env:
            raise OverflowError("Rollout buffer overflow! You should call clear() before adding new transitions.")
        s = self.step
        for k in self.observations:
            self.observations[k][s].copy_(t.observations[k])
        self.actions[s].copy_(t.actions)
        self.rewards[s].copy_(t.rewards.view(-1, 1))
        self.dones[s].copy_(t.dones.view(-1, 1))
        self.values[s].copy_(t.values)
        self.actions_log_prob[s].copy_(t.actions_log_prob.view(-1, 1))
        if self.distribution_params is None:
            self.distribution_params = tuple(torch.zeros(self.num_transitions_per_env, *p.shape)
                                             for p in t.distribution_params)
        for i, p in enumerate(t.distribution_params):
            self.distribution_params[i][s].copy_(p)
        self._save_hidden_states(t.hidden_states)
        self.step += 1

    def clear(self) -> None:
        self.step = 0

    def mini_batch_generator(self, num_mini_batches: int, num_epochs: int = 8):
        """rollout_storage.py:225-259: ONE randperm per call, reused by every epoch; rows are t*N + n."""
        batch_size = self.num_envs * self.num_transitions_per_env
        if not 1 <= num_mini_batches <= batch_size:
            raise ValueError("num_mini_batches must be between 1 and the rollout batch size.")
        indices = torch.randperm(batch_size, requires_grad=False)
        obs = {k: v.flatten(0, 1) for k, v in self.observations.items()}
        actions = self.actions.flatten(0, 1)
        values = self.values.flatten(0, 1)
        returns = self.returns.flatten(0, 1)
        old_logp = self.actions_log_prob.flatten(0, 1)
        advantages = self.advantages.flatten(0, 1)
        old_params = tuple(p.flatten(0, 1) for p in self.distribution_params)
        for _ in range(num_epochs):
            for i in range(num_mini_batches):
                idx = indices[i * batch_size // num_mini_batches:(i + 1) * batch_size // num_mini_batches]
                yield Batch(
                    observations={k: v[idx] for k, v in obs.items()},
                    actions=actions[idx],
                    values=values[idx],
                    advantages=advantages[idx],
                    returns=returns[idx],
                    old_actions_log_prob=old_logp[idx],
                    old_distribution_params=tuple(p[idx] for p in old_params),
                    indices=idx,
                )

    def recurrent_mini_batch_generator(self, num_mini_batches: int, num_epochs: int = 8):
        """rollout_storage.py:262-331: env slices, no shuffling, trajectories padded at dones."""
        if not 1 <= num_mini_batches <= self.num_envs:
            raise ValueError("num_mini_batches must be between 1 and the number of environments.")
        padded_obs, traj_masks = split_and_pad_trajectories(self.observations, self.dones)
        for _ in range(num_epochs):
            first_traj = 0
            for i in range(num_mini_batches):
                start = i * self.num_envs // num_mini_batches
                stop = (i + 1) * self.num_envs // num_mini_batches
                dones = self.dones.squeeze(-1)
                last_was_done = torch.zeros_like(dones, dtype=torch.bool)
                last_was_done[1:] = dones[:-1]
                last_was_done[0] = True
                last_traj = first_traj + int(torch.sum(last_was_done[:, start:stop]))
                starts = last_was_done.permute(1, 0)

                def pick(saved):
                    if saved is None:
                        return None
                    hs = [h.permute(2, 0, 1, 3)[starts][first_traj:last_traj].transpose(1, 0).contiguous()
                          for h in saved]
                    return hs[0] if len(hs) == 1 else tuple(hs)

                yield Batch(
                    observations={k: v[:, first_traj:last_traj] for k, v in padded_obs.items()},
                    actions=self.actions[:, start:stop],
                    values=self.values[:, start:stop],
                    advantages=self.advantages[:, start:stop],
                    returns=self.returns[:, start:stop],
                    old_actions_log_prob=self.actions_log_prob[:, start:stop],
                    old_distribution_params=tuple(p[:, start:stop] for p in self.distribution_params),
                    hidden_states=(pick(self.saved_hidden_state_a), pick(self.saved_hidden_state_c)),
                    masks=traj_masks[:, first_traj:last_traj],
                )
                first_traj = last_traj

    def _save_hidden_states(self, hidden_states) -> None:
        """rollout_storage.py:333-359."""
        if hidden_states == (None, None) or hidden_states is None:
            return
        T = self.num_transitions_per_env
        ha = hidden_states[0] if isinstance(hidden_states[0], tuple) else (hidden_states[0],)
        hc = hidden_states[1] if isinstance(hidden_states[1], tuple) else (hidden_states[1],)
        if self.saved_hidden_state_a is None and hidden_states[0] is not None:
            self.saved_hidden_state_a = [torch.zeros(T, *h.shape) for h in ha]
        if self.saved_hidden_state_c is None and hidden_states[1] is not None:
            self.saved_hidden_state_c = [torch.zeros(T, *h.shape) for h in hc]
        if hidden_states[0] is not None:
            for i, h in enumerate(ha):
                self.saved_hidden_state_a[i][self.step].copy_(h)
        if hidden_states[1] is not None:
            for i, h in enumerate(hc):
                self.saved_hidden_state_c[i][self.step].copy_(h)


# ----------------------------------------------------------------------------------------------------------------------
# the arithmetic blocks of PPO, as standalone functions (PPO below calls exactly these)
# ----------------------------------------------------------------------------------------------------------------------


def gae_returns(rewards, values, dones, last_values, gamma: float, lam: float, normalize: bool = True):
    """ppo.py:175-191 on [T, N, 1] tensors: reverse-time GAE, advantages = returns - values, then (optionally) the
    global normalisation with the unbiased std and eps outside the sqrt."""
    T = rewards.shape[0]
    returns = torch.zeros_like(rewards)
    advantage = 0
    for step in reversed(range(T)):
        next_values = last_values if step == T - 1 else values[step + 1]
        not_terminal = 1.0 - dones[step].float()
        delta = rewards[step] + not_terminal * gamma * next_values - values[step]
        advantage = delta + not_terminal * gamma * lam * advantage
        returns[step] = advantage + values[step]
    advantages = returns - values
    if normalize and advantages.numel() > 1:
        advantages = (advantages - advantages.mean()) / (advantages.std() + 1e-8)
    return returns, advantages


def ppo_loss_terms(logp, old_logp, advantages, values, old_values, returns, entropy, clip_param: float,
                   use_clipped_value_loss: bool, value_loss_coef: float, entropy_coef: float, branch=None):
    """ppo.py:268-285: clipped surrogate, (clipped) value loss and the total loss.

    ``branch`` (not upstream; None gives upstream's arithmetic unchanged) is a BranchRecord.  It takes the rows whose
    gradient is zero or not from elsewhere (another implementation's decisions), and records which rows then differ
    from this evaluation's own decision and how far each lies from a clip boundary.  A row that another evaluation
    computes a few ulps differently may fall on the other side of a boundary of max / clamp, where the gradient
    jumps between -adv (or 2 (V - R)) and 0; everywhere else the arithmetic is upstream's."""
    ratio = torch.exp(logp - old_logp.squeeze(-1))
    adv = advantages.squeeze(-1)
    surrogate = -adv * ratio
    lo, hi = 1.0 - clip_param, 1.0 + clip_param
    surrogate_clipped = -adv * torch.clamp(ratio, lo, hi)
    surrogate_rows = torch.max(surrogate, surrogate_clipped)
    if branch is not None:
        with torch.no_grad():
            inside = (ratio >= lo) & (ratio <= hi)
            own = (inside | (surrogate > surrogate_clipped)) & (adv != 0)
            r64 = ratio.double()
            dist = torch.minimum((r64 - hi).abs(), (r64 - lo).abs())
        surrogate_rows = branch.apply("surrogate", surrogate_rows, surrogate, own, dist, ratio)
    surrogate_loss = surrogate_rows.mean()
    if use_clipped_value_loss:
        value_clipped = old_values + (values - old_values).clamp(-clip_param, clip_param)
        value_losses = (values - returns).pow(2)
        value_losses_clipped = (value_clipped - returns).pow(2)
        value_rows = torch.max(value_losses, value_losses_clipped)
        if branch is not None:
            with torch.no_grad():
                dv = (values - old_values).double()
                own = ~((value_losses < value_losses_clipped) & ((dv < -clip_param) | (dv > clip_param)))
                l1, l2 = value_losses.double(), value_losses_clipped.double()
                # the gradient is zero or not depending on the clamp edge and on which square is larger
                dist = torch.minimum((dv - clip_param).abs(), (dv + clip_param).abs())
                gap = (l1 - l2).abs() / torch.maximum(l1, l2).clamp(min=1e-30)
            value_rows = branch.apply("value", value_rows, value_losses, own, dist, values,
                                      {"gap": gap, "err": (values - returns).double().abs()})
        value_loss = value_rows.mean()
    else:
        value_loss = (returns - values).pow(2).mean()
    loss = surrogate_loss + value_loss_coef * value_loss - entropy_coef * entropy.mean()
    return surrogate_loss, value_loss, loss


class BranchRecord:
    """Per mini-batch record of the clip branches (not upstream; see ppo_loss_terms).

    ``forced``: kind ("surrogate" / "value") -> bool tensor of the rows whose gradient must be non-zero, in the
    mini-batch's row order (None: keep this evaluation's own decisions).  After the loss is built, ``own[kind]``
    holds this evaluation's decisions, ``q[kind]`` the quantity they depend on (the ratio, the value V; fp64 copies)
    and ``flips[kind]`` = (rows, distance to the boundary) of the rows where the forced decision differs from the own
    one: |ratio - (1 +- clip)| for the surrogate, |(V - V_old) -+ clip| for the value loss, whose rows also carry
    ``extra["value"]``: "gap" = |l1 - l2| / max(l1, l2) of the two squares and "err" = |V - R|."""

    def __init__(self, forced: dict | None = None) -> None:
        self.forced = forced or {}
        self.own: dict = {}
        self.q: dict = {}
        self.extra: dict = {}
        self.flips: dict = {}

    def apply(self, kind: str, rows, active, own, dist, q, extra: dict | None = None):
        """rows: the per-row loss term; active: the term whose gradient a forced non-zero row takes."""
        self.own[kind] = own.reshape(-1).clone()
        self.q[kind] = q.detach().reshape(-1).double().clone()
        if extra is not None:
            self.extra[kind] = {k: v.reshape(-1).clone() for k, v in extra.items()}
        forced = self.forced.get(kind)
        if forced is None:
            self.flips[kind] = (torch.zeros(0, dtype=torch.int64), torch.zeros(0, dtype=torch.float64))
            return rows
        forced = forced.reshape(own.shape).to(torch.bool)
        off = own & ~forced   # this evaluation's gradient is non-zero, the other's zero
        on = ~own & forced    # and the reverse
        idx = torch.nonzero((off | on).reshape(-1)).reshape(-1)
        self.flips[kind] = (idx, dist.reshape(-1)[idx].clone())
        if idx.numel() == 0:
            return rows
        return torch.where(off, rows.detach(), torch.where(on, active, rows))


def adaptive_lr(kl_mean: torch.Tensor, learning_rate: float, desired_kl: float) -> float:
    """ppo.py:253-256 (comparisons of the fp32 tensor against Python floats, LR arithmetic in Python floats)."""
    if kl_mean > desired_kl * 2.0:
        return max(1e-5, learning_rate / 1.5)
    if kl_mean < desired_kl / 2.0 and kl_mean > 0.0:
        return min(1e-2, learning_rate * 1.5)
    return learning_rate


# ----------------------------------------------------------------------------------------------------------------------
# algorithm (rsl_rl/algorithms/ppo.py)
# ----------------------------------------------------------------------------------------------------------------------


def resolve_optimizer(name: str):
    """rsl_rl/utils/utils.py:71-96: the torch optimiser class of a name (adam, adamw, sgd, rmsprop; any case)."""
    table = {"adam": torch.optim.Adam, "adamw": torch.optim.AdamW, "sgd": torch.optim.SGD,
             "rmsprop": torch.optim.RMSprop}
    name = name.lower()
    if name not in table:
        raise ValueError(f"Invalid optimizer '{name}'. Valid optimizers are: {list(table.keys())}")
    return table[name]


class PPO:
    """rsl_rl/algorithms/ppo.py:27-465 on one CPU process (no RND, no symmetry, no multi-GPU)."""

    def __init__(self, actor: MLPModel, critic: MLPModel, storage: RolloutStorage, num_learning_epochs: int = 5,
                 num_mini_batches: int = 4, clip_param: float = 0.2, gamma: float = 0.99, lam: float = 0.95,
                 value_loss_coef: float = 1.0, entropy_coef: float = 0.01, learning_rate: float = 0.001,
                 max_grad_norm: float = 1.0, optimizer: str = "adam", use_clipped_value_loss: bool = True,
                 schedule: str = "adaptive", desired_kl: float = 0.01,
                 normalize_advantage_per_mini_batch: bool = False, use_mixed_precision: bool = False,
                 device: str = "cpu", rnd_cfg=None, symmetry_cfg=None, multi_gpu_cfg=None,
                 grad_reduce_bucket_mb: float = 25) -> None:
        if rnd_cfg or symmetry_cfg or multi_gpu_cfg is not None:
            raise NotImplementedError("RND, symmetry and multi-GPU are outside this oracle")
        self.device = "cpu"
        self.actor = actor
        self.critic = critic
        self.optimizer = resolve_optimizer(optimizer)(
            list(dict.fromkeys(chain(actor.parameters(), critic.parameters()))), lr=learning_rate)
        self.storage = storage
        self.transition = Transition()
        self.clip_param = clip_param
        self.num_learning_epochs = num_learning_epochs
        self.num_mini_batches = num_mini_batches
        self.value_loss_coef = value_loss_coef
        self.entropy_coef = entropy_coef
        self.gamma = gamma
        self.lam = lam
        self.max_grad_norm = max_grad_norm
        self.use_clipped_value_loss = use_clipped_value_loss
        self.desired_kl = desired_kl
        self.schedule = schedule
        self.learning_rate = learning_rate
        self.normalize_advantage_per_mini_batch = normalize_advantage_per_mini_batch
        self.use_mixed_precision = use_mixed_precision
        # per-mini-batch diagnostics (not upstream): kl_mean, lr after the rule, the three losses, batch indices
        self.trace: list[dict] = []
        # per-mini-batch state hook (not upstream): called as recorder("pre", self) before a mini-batch's forward
        # pass and recorder("post", self) after its optimiser step; tests use it to snapshot the training state
        self.recorder = None
        # per-mini-batch clip-branch decisions to take from another evaluation (not upstream): a list with one dict
        # kind -> bool rows (or None) per optimiser step; see BranchRecord.  The trace then reports the flipped rows.
        self.forced_branches: list | None = None
        # stop after this many optimiser steps (not upstream; tests that check only the first steps of a large update)
        self.max_steps: int | None = None

    # -- rollout side ------------------------------------------------------------------------------------------------
    def act(self, obs: Mapping) -> torch.Tensor:
        """ppo.py:124-135."""
        self.transition.hidden_states = (self.actor.get_hidden_state(), self.critic.get_hidden_state())
        self.transition.actions = self.actor(obs, stochastic_output=True).detach()
        self.transition.values = self.critic(obs).detach()
        self.transition.actions_log_prob = self.actor.get_output_log_prob(self.transition.actions).detach()
        self.transition.distribution_params = tuple(p.detach() for p in self.actor.output_distribution_params)
        self.transition.observations = obs
        return self.transition.actions

    def process_env_step(self, obs: Mapping, rewards: torch.Tensor, dones: torch.Tensor, extras: dict) -> None:
        """ppo.py:137-164."""
        self.transition.rewards = rewards.clone()
        self.transition.dones = dones
        if "time_outs" in extras:
            self.transition.rewards += self.gamma * torch.squeeze(
                self.transition.values * extras["time_outs"].unsqueeze(1), 1)
        self.storage.add_transition(self.transition)
        self.transition.clear()
        self.actor.reset(dones)
        self.critic.reset(dones)

    def compute_returns(self, obs: Mapping, last_values: torch.Tensor | None = None) -> None:
        """ppo.py:166-191.  ``last_values`` (not upstream) replaces the critic bootstrap, as upstream's own GAE tests
        do by monkeypatching ``critic.forward`` (tests/algorithms/test_ppo.py:182-184)."""
        st = self.storage
        if last_values is None:
            hidden = self.critic.get_hidden_state()
            last_values = self.critic(obs).detach()
            self.critic.reset(hidden_state=hidden)
        st.returns, st.advantages = gae_returns(st.rewards, st.values, st.dones, last_values, self.gamma, self.lam,
                                                normalize=not self.normalize_advantage_per_mini_batch)

    # -- learning side -----------------------------------------------------------------------------------------------
    def update(self) -> dict[str, float]:
        """ppo.py:193-358."""
        mean_value_loss = 0.0
        mean_surrogate_loss = 0.0
        mean_entropy = 0.0
        self.trace = []
        for batch in self.batches():
            if self.max_steps is not None and len(self.trace) >= self.max_steps:
                break
            if self.recorder is not None:
                self.recorder("pre", self)
            k = len(self.trace)
            forced = self.forced_branches[k] if self.forced_branches is not None else None
            t = self.minibatch_step(batch, forced)
            if self.recorder is not None:
                self.recorder("post", self)
            mean_value_loss += t["value"]
            mean_surrogate_loss += t["surrogate"]
            mean_entropy += t["entropy"]
            self.trace.append(t)
        obs = {k: v.flatten(0, 1) for k, v in self.storage.observations.items()}
        self.actor.update_normalization(obs)
        self.critic.update_normalization(obs)
        n = self.num_learning_epochs * self.num_mini_batches
        self.storage.clear()
        return {"value": mean_value_loss / n, "surrogate": mean_surrogate_loss / n, "entropy": mean_entropy / n}

    def batches(self):
        """The mini-batches update() iterates (ppo.py:204-208): one randperm per call for feed-forward models."""
        if self.actor.is_recurrent or self.critic.is_recurrent:
            return self.storage.recurrent_mini_batch_generator(self.num_mini_batches, self.num_learning_epochs)
        return self.storage.mini_batch_generator(self.num_mini_batches, self.num_learning_epochs)

    def minibatch_step(self, batch, forced: dict | None = None) -> dict:
        """The body of update()'s loop for one mini-batch (ppo.py:210-319): losses, backward, per-model clipping,
        Adam.  Returns the trace entry of the step.  ``forced``: see ``forced_branches``."""
        if self.normalize_advantage_per_mini_batch and batch.advantages.numel() > 1:
            with torch.no_grad():
                batch.advantages = (batch.advantages - batch.advantages.mean()) / (batch.advantages.std() + 1e-8)
        branch = BranchRecord(forced)
        with torch.amp.autocast(device_type="cpu", enabled=self.use_mixed_precision, dtype=torch.bfloat16):
            self.actor(batch.observations, masks=batch.masks, hidden_state=batch.hidden_states[0],
                       stochastic_output=True)
            logp = self.actor.get_output_log_prob(batch.actions)
            values = self.critic(batch.observations, masks=batch.masks, hidden_state=batch.hidden_states[1])
            dist_params = self.actor.output_distribution_params
            entropy = self.actor.output_entropy
            kl_value = None
            if self.desired_kl is not None and self.schedule == "adaptive":
                with torch.inference_mode():
                    kl = self.actor.get_kl_divergence(batch.old_distribution_params, dist_params)
                    kl_mean = torch.mean(kl)
                    kl_value = float(kl_mean)
                    self.learning_rate = adaptive_lr(kl_mean, self.learning_rate, self.desired_kl)
                    for group in self.optimizer.param_groups:
                        group["lr"] = self.learning_rate
            surrogate_loss, value_loss, loss = ppo_loss_terms(
                logp, batch.old_actions_log_prob, batch.advantages, values, batch.values, batch.returns, entropy,
                self.clip_param, self.use_clipped_value_loss, self.value_loss_coef, self.entropy_coef, branch)
        self.optimizer.zero_grad()
        loss.backward()
        nn.utils.clip_grad_norm_(self.actor.parameters(), self.max_grad_norm)
        nn.utils.clip_grad_norm_(self.critic.parameters(), self.max_grad_norm)
        self.optimizer.step()
        with torch.no_grad():  # diagnostic: distance of the nearest ratio to a clip boundary (not upstream)
            ratio = torch.exp(logp.detach() - batch.old_actions_log_prob.squeeze(-1)).double()
            margin = torch.minimum((ratio - (1.0 + self.clip_param)).abs(),
                                   (ratio - (1.0 - self.clip_param)).abs()).min().item()
        return {"kl_mean": kl_value, "lr": self.learning_rate, "value": value_loss.item(),
                "surrogate": surrogate_loss.item(), "entropy": entropy.mean().item(), "indices": batch.indices,
                "clip_margin": margin, "branches": branch}

    def train_mode(self) -> None:
        self.actor.train()
        self.critic.train()

    def eval_mode(self) -> None:
        self.actor.eval()
        self.critic.eval()

    def save(self) -> dict:
        """ppo.py:374-385."""
        return {"actor_state_dict": self.actor.state_dict(), "critic_state_dict": self.critic.state_dict(),
                "optimizer_state_dict": self.optimizer.state_dict()}


def _model_class(name):
    short = name.split(":")[-1].split(".")[-1] if isinstance(name, str) else name.__name__
    if short == "MLPModel":
        return MLPModel
    if short == "RNNModel":
        return RNNModel
    raise NotImplementedError(f"model class {name} is not on the PPO path of this oracle")


def construct_algorithm(obs: Mapping, num_envs: int, num_actions: int, cfg: dict) -> PPO:
    """ppo.py:428-465 without class resolution (the oracle only knows its own classes).  RNG order: actor then critic
    default ``nn.Linear`` initialisation, exactly as upstream."""
    alg_cfg = dict(cfg["algorithm"])
    alg_cfg.pop("class_name", None)
    actor_cfg = dict(cfg["actor"])
    critic_cfg = dict(cfg["critic"])
    actor_cls = _model_class(actor_cfg.pop("class_name", "MLPModel"))
    critic_cls = _model_class(critic_cfg.pop("class_name", "MLPModel"))
    groups = resolve_obs_groups(obs, dict(cfg.get("obs_groups", {})), ["actor", "critic"])
    cfg["obs_groups"] = groups
    actor = actor_cls(obs, groups, "actor", num_actions, **actor_cfg)
    critic = critic_cls(obs, groups, "critic", 1, **critic_cfg)
    storage = RolloutStorage(num_envs, cfg["num_steps_per_env"], obs, [num_actions])
    return PPO(actor, critic, storage, **alg_cfg)


def gae_fp64(rewards, values, dones, last_values, gamma: float, lam: float):
    """Textbook GAE in float64 (independent of upstream's op order): A_t = d_t + g*l*(1-done_t)*A_{t+1},
    d_t = r_t + g*(1-done_t)*V_{t+1} - V_t, R_t = A_t + V_t.  Inputs [T, N]."""
    r = np.asarray(rewards, dtype=np.float64)
    v = np.asarray(values, dtype=np.float64)
    d = np.asarray(dones, dtype=np.float64)
    lv = np.asarray(last_values, dtype=np.float64).reshape(-1)
    T = r.shape[0]
    ret = np.zeros_like(r)
    adv = np.zeros(r.shape[1])
    for t in range(T - 1, -1, -1):
        nv = lv if t == T - 1 else v[t + 1]
        nt = 1.0 - d[t]
        delta = r[t] + gamma * nt * nv - v[t]
        adv = delta + gamma * lam * nt * adv
        ret[t] = adv + v[t]
    return ret, ret - v


def math_log_sqrt_2pi() -> float:
    return math.log(math.sqrt(2 * math.pi))
