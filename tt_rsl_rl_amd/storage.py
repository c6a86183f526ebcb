"""Device-resident rollout storage with upstream's layout and interface (rsl_rl/storage/rollout_storage.py:17-359).

Buffers are [T, N, ...] time-major tensors in HBM, exactly upstream's shapes (observations per group, actions,
rewards, uint8 dones, values, log-probs, distribution params (mean, std), returns, advantages), so a flat row index
is t * N + n as upstream's ``flatten(0, 1)``.  The PPO plugin's update reads them through the packed-table gather
kernel; ``mini_batch_generator`` is kept for API compatibility (it yields the same mini-batches upstream would).
"""

from __future__ import annotations

from typing import Mapping

import torch


class RolloutStorage:
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
            self.privileged_actions = None
            self.hidden_states = (None, None)

        def clear(self) -> None:
            self.__init__()

    class Batch:
        """rollout_storage.py:67-123."""

        def __init__(self, observations=None, actions=None, values=None, advantages=None, returns=None,
                     old_actions_log_prob=None, old_distribution_params=None, hidden_states=(None, None), masks=None,
                     privileged_actions=None, dones=None) -> None:
            self.observations = observations
            self.actions = actions
            self.values = values
            self.advantages = advantages
            self.returns = returns
            self.old_actions_log_prob = old_actions_log_prob
            self.old_distribution_params = old_distribution_params
            self.hidden_states = hidden_states
            self.masks = masks
            self.privileged_actions = privileged_actions
            self.dones = dones

    def __init__(self, training_type: str, num_envs: int, num_transitions_per_env: int, obs: Mapping,
                 actions_shape, device: str = "cuda") -> None:
        if training_type != "rl":
            raise NotImplementedError("only training_type='rl' is on the PPO update path")
        self.training_type = training_type
        self.device = torch.device(device)
        self.num_transitions_per_env = T = num_transitions_per_env
        self.num_envs = N = num_envs
        self.actions_shape = list(actions_shape)
        self.observations = {k: torch.zeros(T, *v.shape, dtype=v.dtype, device=self.device) for k, v in obs.items()}
        self.rewards = torch.zeros(T, N, 1, device=self.device)
        self.actions = torch.zeros(T, N, *actions_shape, device=self.device)
        self.dones = torch.zeros(T, N, 1, device=self.device).byte()
        self.values = torch.zeros(T, N, 1, device=self.device)
        self.actions_log_prob = torch.zeros(T, N, 1, device=self.device)
        self.distribution_params: tuple[torch.Tensor, ...] | None = None
        self.returns = torch.zeros(T, N, 1, device=self.device)
        self.advantages = torch.zeros(T, N, 1, device=self.device)
        self.saved_hidden_state_a = None
        self.saved_hidden_state_c = None
        self.step = 0

    def add_transition(self, transition: "RolloutStorage.Transition") -> None:
        """rollout_storage.py:173-205 (copies into the device buffers)."""
        if self.step >= self.num_transitions_per_env:
            raise OverflowError("Rollout buffer overflow! You should call clear() before adding new transitions.")
        s = self.step
        for k in self.observations:
            self.observations[k][s].copy_(transition.observations[k])
        self.actions[s].copy_(transition.actions)
        self.rewards[s].copy_(transition.rewards.view(-1, 1))
        self.dones[s].copy_(transition.dones.view(-1, 1))
        self.values[s].copy_(transition.values)
        self.actions_log_prob[s].copy_(transition.actions_log_prob.view(-1, 1))
        if self.distribution_params is None:
            self.distribution_params = tuple(
                torch.zeros(self.num_transitions_per_env, *p.shape, device=self.device)
                for p in transition.distribution_params)
        for i, p in enumerate(transition.distribution_params):
            self.distribution_params[i][s].copy_(p)
        self._save_hidden_states(transition.hidden_states)
        self.step += 1

    def _save_hidden_states(self, hidden_states) -> None:
        """rollout_storage.py:333-359: the recurrent models' state before each step's forward, as saved_hidden_state_a /
        _c = [h, c] each [T, num_layers, N, H] (zero where a model had no state yet)."""
        if hidden_states is None or hidden_states == (None, None):
            return
        T = self.num_transitions_per_env
        for side, hs in (("a", hidden_states[0]), ("c", hidden_states[1])):
            if hs is None:
                continue
            hs = hs if isinstance(hs, tuple) else (hs,)
            name = f"saved_hidden_state_{side}"
            if getattr(self, name) is None:
                setattr(self, name, [torch.zeros(T, *h.shape, device=self.device) for h in hs])
            for buf, h in zip(getattr(self, name), hs):
                buf[self.step].copy_(h)

    def clear(self) -> None:
        self.step = 0

    @property
    def batch_size(self) -> int:
        return self.num_envs * self.num_transitions_per_env

    def flat(self, t: torch.Tensor) -> torch.Tensor:
        """[T, N, ...] -> [T*N, width] row-major view (row = t*N + n)."""
        return t.reshape(self.batch_size, -1)

    def mini_batch_generator(self, num_mini_batches: int, num_epochs: int = 8):
        """rollout_storage.py:225-259 (API compatibility; one randperm on the CPU generator, reused by every epoch)."""
        B = self.batch_size
        if not 1 <= num_mini_batches <= B:
            raise ValueError("num_mini_batches must be between 1 and the rollout batch size.")
        indices = torch.randperm(B).to(self.device)
        obs = {k: v.flatten(0, 1) for k, v in self.observations.items()}
        fields = [self.actions.flatten(0, 1), self.values.flatten(0, 1), self.advantages.flatten(0, 1),
                  self.returns.flatten(0, 1), self.actions_log_prob.flatten(0, 1)]
        params = tuple(p.flatten(0, 1) for p in self.distribution_params)
        for _ in range(num_epochs):
            for i in range(num_mini_batches):
                idx = indices[i * B // num_mini_batches:(i + 1) * B // num_mini_batches]
                a, v, adv, ret, lp = (f[idx] for f in fields)
                yield RolloutStorage.Batch(observations={k: o[idx] for k, o in obs.items()}, actions=a, values=v,
                                           advantages=adv, returns=ret, old_actions_log_prob=lp,
                                           old_distribution_params=tuple(p[idx] for p in params))

    def recurrent_mini_batch_generator(self, num_mini_batches: int, num_epochs: int = 8):
        """Not provided: the update evaluates upstream's padded trajectories in the equivalent masked per-env form on
        the GPU (one sequence per env from saved_hidden_state_*[0], state zeroed after every done)."""
        raise NotImplementedError("the recurrent update does not materialise padded trajectories")
