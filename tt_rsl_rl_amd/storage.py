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
        # actions and the distribution parameters as column blocks of one record per transition (set up at the first
        # transition, when the parameters' shapes are known): see _interleave
        self.act_record: torch.Tensor | None = None
        self.act_record_pad = 0
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
        if self.distribution_params is None:
            self._interleave(transition.distribution_params)
        for k in self.observations:
            self.observations[k][s].copy_(transition.observations[k])
        self.actions[s].copy_(transition.actions)
        self.rewards[s].copy_(transition.rewards.view(-1, 1))
        self.dones[s].copy_(transition.dones.view(-1, 1))
        self.values[s].copy_(transition.values)
        self.actions_log_prob[s].copy_(transition.actions_log_prob.view(-1, 1))
        for i, p in enumerate(transition.distribution_params):
            self.distribution_params[i][s].copy_(p)
        self._save_hidden_states(transition.hidden_states)
        self.step += 1

    def _interleave(self, params) -> None:
        """Storage for the actions and the distribution parameters.  When every parameter has the actions' [N, A]
        shape (a Gaussian's mean and std), they are column blocks of one record per transition, [T, N, k * Ap] with
        block i at columns i * Ap .. i * Ap + A (Ap = A rounded up to 4, zero padding between), and ``actions`` /
        ``distribution_params`` are views of it with upstream's shapes: the update's gather then reads one
        contiguous record per sampled row instead of k scattered short rows (each of which pulls whole cache lines).
        Otherwise separate [T, N, ...] buffers as upstream allocates them."""
        T, N = self.num_transitions_per_env, self.num_envs
        if len(self.actions_shape) == 1 and all(tuple(p.shape) == (N, self.actions_shape[0]) for p in params):
            A = self.actions_shape[0]
            ap = -(-A // 4) * 4
            rec = torch.zeros(T, N, (1 + len(params)) * ap, device=self.device)
            self.act_record, self.act_record_pad = rec, ap
            self.actions = rec[..., :A]
            self.distribution_params = tuple(rec[..., (i + 1) * ap:(i + 1) * ap + A] for i in range(len(params)))
        else:
            self.distribution_params = tuple(torch.zeros(T, *p.shape, device=self.device) for p in params)

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
        """rollout_storage.py:262-331 (API compatibility; the update itself evaluates the same trajectories in the
        masked per-env form on the GPU).  Mini-batch i is the env slice [i N / M, (i + 1) N / M), all steps, the same
        slices every epoch: its observations as trajectories split at the dones and zero-padded to T steps
        ([T, trajectories, ...], rsl_rl/utils/utils.py:395-449, trajectories in env-major order), the masks of their
        valid steps, the state each trajectory starts from, and the other fields unpadded [T, envs, ...]."""
        if not 1 <= num_mini_batches <= self.num_envs:
            raise ValueError("num_mini_batches must be between 1 and the number of environments.")
        padded_obs, masks, starts = self._padded_trajectories()
        starts_env_major = starts.transpose(1, 0)  # [N, T]: which (env, step) begin a trajectory
        # trajectories of env slice [0, e): every start of those envs (counted env-major)
        starts_per_env = starts_env_major.sum(dim=1).cumsum(0).tolist()

        def states(saved):
            if saved is None:
                return None
            # [T, layers, N, H] -> the states at the trajectory starts, env-major -> [layers, trajectories, H]
            picked = [h.permute(2, 0, 1, 3)[starts_env_major] for h in saved]
            return picked

        sa, sc = states(self.saved_hidden_state_a), states(self.saved_hidden_state_c)

        def select(picked, t0, t1):
            if picked is None:
                return None
            out = [p[t0:t1].transpose(1, 0).contiguous() for p in picked]
            return out[0] if len(out) == 1 else tuple(out)

        for _ in range(num_epochs):
            for i in range(num_mini_batches):
                start = i * self.num_envs // num_mini_batches
                stop = (i + 1) * self.num_envs // num_mini_batches
                first = starts_per_env[start - 1] if start > 0 else 0
                last = starts_per_env[stop - 1]
                yield RolloutStorage.Batch(
                    observations={k: v[:, first:last] for k, v in padded_obs.items()},
                    actions=self.actions[:, start:stop], values=self.values[:, start:stop],
                    advantages=self.advantages[:, start:stop], returns=self.returns[:, start:stop],
                    old_actions_log_prob=self.actions_log_prob[:, start:stop],
                    old_distribution_params=tuple(p[:, start:stop] for p in self.distribution_params),
                    hidden_states=(select(sa, first, last), select(sc, first, last)),
                    masks=masks[:, first:last])

    def _padded_trajectories(self):
        """The observations split into trajectories at the dones (the last step closes every env's last one) and
        zero-padded to T steps, trajectories in env-major order: [T, trajectories, ...]; the masks of their valid
        steps [T, trajectories]; and the steps that begin a trajectory [T, N] (step 0 and every step after a done)."""
        T, N = self.num_transitions_per_env, self.num_envs
        dones = self.dones[..., 0].bool()
        starts = torch.zeros_like(dones)
        starts[0] = True
        starts[1:] = dones[:-1]
        # env-major numbering: trajectory id of every (env, step), and the step's position inside its trajectory
        se = starts.transpose(1, 0)                                  # [N, T]
        traj = se.reshape(-1).cumsum(0).view(N, T) - 1               # [N, T]
        steps = torch.arange(T, device=dones.device).expand(N, T)
        begin = torch.where(se, steps, torch.zeros_like(steps)).cummax(dim=1).values
        pos = steps - begin                                          # [N, T]
        count = int(se.sum())
        masks = torch.zeros(T, count, dtype=torch.bool, device=dones.device)
        masks[pos.reshape(-1), traj.reshape(-1)] = True
        padded = {}
        for k, v in self.observations.items():
            ve = v.transpose(1, 0).reshape(N * T, *v.shape[2:])
            out = torch.zeros(T, count, *v.shape[2:], dtype=v.dtype, device=v.device)
            out[pos.reshape(-1), traj.reshape(-1)] = ve
            padded[k] = out
        return padded, masks, starts