"""PPO plugin for upstream rsl_rl's OnPolicyRunner, running the update on MI355X through libppo_hip.so.

Selected with ``cfg["algorithm"]["class_name"] = "tt_rsl_rl_amd.ppo:PPO"``; the runner then calls
``PPO.construct_algorithm(obs, env, cfg, device)`` (upstream rsl_rl/algorithms/ppo.py:428-465) and the methods
upstream's runner uses: train_mode / eval_mode / act / process_env_step / compute_returns / update /
learning_rate / get_policy / save / load (rsl_rl/runners/on_policy_runner.py:39-169).

Compatibility kept with upstream:
  * constructor keywords and defaults (ppo.py:40-68); RND / symmetry / multi-GPU raise NotImplementedError;
  * actor / critic / optimizer state_dict layouts: the models keep upstream's module names and parameter order,
    and ``self.optimizer`` is a real ``torch.optim.Adam`` whose state tensors are views of the flat buffers the
    kernels update, so ``save()`` / ``load()`` produce and accept upstream checkpoints;
  * the random stream of upstream's CPU run: the rollout's action noise is drawn from torch's CPU generator, each
    update draws its permutation (``torch.randperm``) from it and then skips the samples upstream's stochastic forward
    draws and discards in every mini-batch, so after the same ``torch.manual_seed`` the actions' noise and every
    update's mini-batch indices are bit-identical to upstream's over any number of iterations
    (``hip_cfg={"rng_stream": "device"}`` draws the rollout noise from the device generator instead and skips no
    samples: the permutation stays on the CPU generator).
"""

from __future__ import annotations

import copy
import importlib
import warnings
from itertools import chain
from typing import Mapping

import torch
import torch.nn as nn

from . import _lib as L
from . import ops
from .engine import RecurrentUpdateEngine, UpdateEngine
from .models import MLPModel, RNNModel
from .storage import RolloutStorage


# ----------------------------------------------------------------------------------------------------------------------
# class resolution (rsl_rl/utils/utils.py:99-189) -- simple names resolve inside this package
# ----------------------------------------------------------------------------------------------------------------------

def resolve_callable(name):
    if callable(name):
        return name
    if not isinstance(name, str):
        raise TypeError(f"Expected callable or string, got {type(name)}")
    short = name.split(":")[-1].split(".")[-1]
    local = {"PPO": PPO, "MLPModel": MLPModel, "RNNModel": RNNModel, "RolloutStorage": RolloutStorage}
    if ":" in name:
        mod, attr = name.rsplit(":", 1)
        if mod.split(".")[0] == "rsl_rl" and short in local:
            return local[short]  # upstream's classes map onto their HIP counterparts
        obj = importlib.import_module(mod)
        for a in attr.split("."):
            obj = getattr(obj, a)
        return obj
    if short in local:
        return local[short]
    raise ValueError(f"Could not resolve '{name}'. Use a qualified name like 'module.path:ClassName'.")


def resolve_class(cfg: dict):
    c = copy.deepcopy(cfg)
    return resolve_callable(c.pop("class_name")), c


def resolve_obs_groups(obs: Mapping, obs_groups: dict, default_sets: list[str]) -> dict:
    """rsl_rl/utils/utils.py:192-287."""
    if len(obs_groups) == 0:
        warnings.warn("The observation configuration dictionary 'obs_groups' is empty and thus likely not configured.")
    else:
        for set_name, groups in obs_groups.items():
            if len(groups) == 0:
                raise ValueError(f"The '{set_name}' key in the 'obs_groups' dictionary can not be an empty list.")
            for g in groups:
                if g not in obs:
                    raise ValueError(f"Observation '{g}' in observation set '{set_name}' not found in the observations "
                                     f"from the environment. Available observations: {list(obs.keys())}")
    for name in default_sets:
        if name not in obs_groups:
            if name in obs:
                obs_groups[name] = [name]
            elif "policy" in obs:
                obs_groups[name] = ["policy"]
            else:
                raise ValueError(f"The observation configuration dictionary 'obs_groups' does not contain the '{name}'"
                                 " key and no suitable observation could be found.")
    return obs_groups


# ----------------------------------------------------------------------------------------------------------------------
# flat parameter buffers
# ----------------------------------------------------------------------------------------------------------------------

class FlatParams:
    """Parameters, gradients and Adam moments of an ordered parameter list as views of four flat fp32 buffers.

    Every parameter starts on a 64-byte boundary (ALIGN floats) so the GEMM kernels can fetch weight rows with
    16-byte loads; the zero padding between parameters has zero gradient and stays zero under Adam."""

    ALIGN = 16

    def __init__(self, groups: list[list[nn.Parameter]], device) -> None:
        params = [p for g in groups for p in g]
        a = self.ALIGN
        n = sum(-(-p.numel() // a) * a for p in params)
        self.param = torch.zeros(n, device=device)
        self.grad = torch.zeros(n, device=device)
        self.exp_avg = torch.zeros(n, device=device)
        self.exp_avg_sq = torch.zeros(n, device=device)
        self.offsets: dict[int, tuple[int, int]] = {}
        bounds = [0]
        off = 0
        with torch.no_grad():
            for g in groups:
                for p in g:
                    k = p.numel()
                    self.param[off:off + k].copy_(p.detach().reshape(-1))
                    p.data = self.param[off:off + k].view(p.shape)
                    p.grad = self.grad[off:off + k].view(p.shape)
                    self.offsets[id(p)] = (off, k)
                    off += -(-k // a) * a
                bounds.append(off)
        self.group_begin = torch.tensor(bounds, dtype=torch.int64)
        self.params = params

    def _view(self, buf: torch.Tensor, p: nn.Parameter) -> torch.Tensor:
        off, k = self.offsets[id(p)]
        return buf[off:off + k].view(p.shape)

    def grad_view(self, p: nn.Parameter) -> torch.Tensor:
        return self._view(self.grad, p)

    def exp_avg_view(self, p: nn.Parameter) -> torch.Tensor:
        return self._view(self.exp_avg, p)

    def exp_avg_sq_view(self, p: nn.Parameter) -> torch.Tensor:
        return self._view(self.exp_avg_sq, p)


# ----------------------------------------------------------------------------------------------------------------------
# the algorithm
# ----------------------------------------------------------------------------------------------------------------------

class PPO:
    """Proximal Policy Optimization with the update on the GPU (upstream rsl_rl/algorithms/ppo.py:27-486)."""

    actor: MLPModel
    critic: MLPModel

    def __init__(self, actor: MLPModel, critic: MLPModel, storage: RolloutStorage, num_learning_epochs: int = 5,
                 num_mini_batches: int = 4, clip_param: float = 0.2, gamma: float = 0.99, lam: float = 0.95,
                 value_loss_coef: float = 1.0, entropy_coef: float = 0.01, learning_rate: float = 0.001,
                 max_grad_norm: float = 1.0, optimizer: str = "adam", use_clipped_value_loss: bool = True,
                 schedule: str = "adaptive", desired_kl: float = 0.01,
                 normalize_advantage_per_mini_batch: bool = False, use_mixed_precision: bool = False,
                 device: str = "cuda", rnd_cfg: dict | None = None, symmetry_cfg: dict | None = None,
                 multi_gpu_cfg: dict | None = None, grad_reduce_bucket_mb: float = 25,
                 hip_cfg: dict | None = None) -> None:
        if rnd_cfg:
            raise NotImplementedError("RND is not on the HIP PPO path")
        if symmetry_cfg:
            raise NotImplementedError("symmetry augmentation is not on the HIP PPO path")
        if multi_gpu_cfg is not None:
            raise NotImplementedError("multi-GPU training is not implemented by the HIP PPO plugin (single GPU)")
        if optimizer.lower() not in L.OPTIMIZERS:  # upstream's resolve_optimizer (rsl_rl/utils/utils.py:71-96)
            raise ValueError(f"Invalid optimizer '{optimizer.lower()}'. Valid optimizers are: {list(L.OPTIMIZERS)}")
        if actor.is_recurrent != critic.is_recurrent:
            raise NotImplementedError("the HIP recurrent update needs both actor and critic recurrent (or neither)")
        if actor.distribution is None:
            raise ValueError("the actor needs a GaussianDistribution (distribution_cfg)")
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("tt_rsl_rl_amd.ppo.PPO runs on a GPU device (no CPU path)")
        self.hip_cfg = dict(hip_cfg or {})
        self.rng_stream = self.hip_cfg.get("rng_stream", "cpu")
        if self.rng_stream not in ("cpu", "device"):
            raise ValueError(f"hip_cfg rng_stream '{self.rng_stream}': 'cpu' or 'device'")
        self.is_multi_gpu = False
        self.gpu_global_rank = 0
        self.gpu_world_size = 1
        self.grad_reduce_bucket_mb = grad_reduce_bucket_mb
        self.rnd = None
        self.symmetry = None

        self.actor = actor.to(self.device)
        self.critic = critic.to(self.device)
        self.actor.distribution.host_noise = self.rng_stream == "cpu"
        self._raw_actor = self.actor
        self._raw_critic = self.critic

        # upstream's optimizer parameter list: actor params then critic params, de-duplicated (ppo.py:100-102)
        actor_params = list(dict.fromkeys(self.actor.parameters()))
        critic_params = [p for p in dict.fromkeys(self.critic.parameters()) if p not in set(actor_params)]
        self.flat = FlatParams([actor_params, critic_params], self.device)
        # upstream passes the learning rate only (ppo.py:99-102): every other hyperparameter is torch's default
        self.optim_kind = L.OPTIMIZERS[optimizer.lower()]
        opt_cls = {L.OPTIM_ADAM: torch.optim.Adam, L.OPTIM_ADAMW: torch.optim.AdamW, L.OPTIM_SGD: torch.optim.SGD,
                   L.OPTIM_RMSPROP: torch.optim.RMSprop}[self.optim_kind]
        self.optimizer = opt_cls(actor_params + critic_params, lr=learning_rate)
        d = self.optimizer.defaults
        if d.get("momentum", 0) != 0 or d.get("centered", False) or d.get("nesterov", False) or d.get("amsgrad", False):
            raise NotImplementedError("optimizer defaults outside the fused update (momentum / centered / amsgrad)")
        if self.optim_kind != L.OPTIM_ADAMW and d.get("weight_decay", 0) != 0:
            raise NotImplementedError("coupled weight decay is outside the fused update")
        self.betas = tuple(d.get("betas", (0.9, 0.999)))
        self.adam_eps = float(d.get("eps", 1e-8))
        self.optim_config = L.OptimConfig(kind=self.optim_kind, beta1=self.betas[0], beta2=self.betas[1],
                                          eps=self.adam_eps, weight_decay=float(d.get("weight_decay", 0.0)),
                                          alpha=float(d.get("alpha", 0.0)))
        self._opt_steps = 0

        self.storage = storage
        self.transition = RolloutStorage.Transition()
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
        self.device_state = ops.new_device_state(learning_rate, self.device)
        self._engine: UpdateEngine | None = None
        self._adv_ws = ops.Workspace(self.device)
        self._perm_host: torch.Tensor | None = None
        self._copy_stream = None  # the permutation's second part goes to the device on it (enqueued by the worker)
        self._rest_copied = None
        self._state_host = ops.pinned_state_buffer()
        self._reset_host = ops.pinned_state_buffer()
        self._trace_rows: list | None = None
        self._step_tensor: torch.Tensor | None = None
        self._saved: dict | None = None  # the state before the current update (_save_state)

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
        """ppo.py:137-164 (time-out bootstrap with the pre-step value V(s_t))."""
        self.transition.rewards = rewards.clone()
        self.transition.dones = dones
        if "time_outs" in extras:
            self.transition.rewards += self.gamma * torch.squeeze(
                self.transition.values * extras["time_outs"].unsqueeze(1).to(self.device), 1)
        self.storage.add_transition(self.transition)
        self.transition.clear()
        self.actor.reset(dones)
        self.critic.reset(dones)

    def compute_returns(self, obs: Mapping) -> None:
        """ppo.py:166-191: bootstrap value, GAE scan and global advantage normalisation on the GPU."""
        critic_hidden_state = self.critic.get_hidden_state()
        last_values = self.critic(obs).detach().contiguous()
        # the bootstrap forward must not advance the critic's rollout state (ppo.py:170-173)
        self.critic.reset(hidden_state=critic_hidden_state)
        self.compute_returns_from(last_values)

    def compute_returns_from(self, last_values: torch.Tensor) -> None:
        st = self.storage
        ops.gae(st.rewards, st.values, st.dones, last_values, st.returns, st.advantages, self.gamma, self.lam)
        n = st.advantages.numel()
        if not self.normalize_advantage_per_mini_batch and n > 1:
            ops.adv_normalize(st.advantages, st.advantages, n, ws=self._adv_ws)

    # -- learning side -----------------------------------------------------------------------------------------------
    @property
    def is_recurrent(self) -> bool:
        return bool(self.actor.is_recurrent)

    def _get_engine(self) -> UpdateEngine:
        e = self._engine
        if e is None or e.B != self.storage.batch_size or e.M != self.num_mini_batches:
            self._engine = e = (RecurrentUpdateEngine if self.is_recurrent else UpdateEngine)(self)
        return e

    def update(self) -> dict[str, float]:
        """ppo.py:193-358."""
        st = self.storage
        B = st.batch_size
        if self.is_recurrent:
            if not 1 <= self.num_mini_batches <= st.num_envs:
                raise ValueError("num_mini_batches must be between 1 and the number of environments.")
        elif not 1 <= self.num_mini_batches <= B:
            raise ValueError("num_mini_batches must be between 1 and the rollout batch size.")
        if st.distribution_params is None:
            raise RuntimeError("update() called before any transition was stored")
        engine = self._get_engine()
        # feed-forward: one permutation of the batch for all epochs (ppo.py:207, rollout_storage.py:210-260);
        # recurrent: fixed env slices, no permutation drawn (rollout_storage.py:262-331).  Then the samples upstream's
        # stochastic forward draws and discards, one [rows, A] Normal sample per mini-batch (mlp_model.py:103-106 via
        # ppo.py:228-233): skipped on the CPU generator by the same worker, beside the GPU update
        discards = engine.discard_sizes() if self.rng_stream == "cpu" else []
        perm, ready, rest, shuffle = None, None, None, None
        if not self.is_recurrent:
            if self._perm_host is None or self._perm_host.numel() != B:
                self._perm_host = torch.empty(B, dtype=torch.int64, pin_memory=True)
                self._perm_dev = torch.empty(B, dtype=torch.int64, device=self.device)
            perm = self._perm_dev
            if self._copy_stream is None:
                self._copy_stream = torch.cuda.Stream(self.device)  # (default priority)
                self._rest_copied = torch.cuda.Event()
            copy_stream, rest_copied, host = self._copy_stream, self._rest_copied, self._perm_host

            def copy_rest(sp):  # on the worker, once perm[sp.split:] is final: its copy, beside the update's kernels
                with torch.cuda.device(self.device), torch.cuda.stream(copy_stream):
                    perm[sp.split:].copy_(host[sp.split:], non_blocking=True)
                    rest_copied.record(copy_stream)

            # torch.randperm(B) on the CPU generator, computed natively (same permutation, same generator state) on a
            # worker thread from here on: the first mini-batch's positions while this thread copies the state and
            # launches the normaliser update below (none of which draws from the generator), then the rest while
            # the first mini-batch's kernels are enqueued
            shuffle = ops.SplitRandperm(B, self._perm_host, engine.minibatch_rows(0)[1], discards, on_rest=copy_rest,
                                        first_on_worker=True)
        try:
            # every update starts from a copy of the state it changes (parameters, Adam moments, normaliser
            # statistics), so an update that fails -- an error raised while its launches are issued, or a device-side
            # failure the read-back reports (the recurrent one-launch sequences) -- leaves the algorithm as it was
            self._save_state()
            # the staging buffer's previous copy (one update ago) completed at that update's read-back
            ops.reset_device_state(self.device_state, self.learning_rate, self._reset_host)
            # The normaliser update (upstream: after the epochs, ppo.py:327-330) reads only the stored raw
            # observations; launched first, on the frozen pre-update statistics the gather uses, it runs while the
            # host draws the permutation.  The epochs see the same statistics as upstream's.
            engine.freeze_normalizers()
            obs = st.observations
            self.actor.update_normalization(obs)
            self.critic.update_normalization(obs)
        except BaseException:
            if shuffle is not None:
                shuffle.join()
            raise
        if self.is_recurrent:
            if discards:
                shuffle = ops.SplitRandperm(0, None, 0, discards)
        else:
            shuffle.wait_first()
            ready = shuffle.split if shuffle.split < B - 1 else B
            perm[:ready].copy_(self._perm_host[:ready], non_blocking=True)
            if ready < B:
                def rest():
                    shuffle.perm_ready()  # (the copy was enqueued on the worker before this returns)
                    torch.cuda.current_stream(self.device).wait_event(rest_copied)
                    consumed[0] = True
        consumed = [False]
        try:
            steps = engine.run(perm, self._opt_steps, ready, rest)
        except BaseException:
            if shuffle is not None:
                shuffle.join()  # idempotent; on an error path it still restores the generator before raising
            if rest is not None and not consumed[0]:
                # the worker may have enqueued the copy of perm[split:] from the pinned host buffer, which the next
                # update's worker rewrites: no stream waits on that copy, so wait for it here
                self._rest_copied.synchronize()
            torch.cuda.current_stream(self.device).synchronize()
            self._restore_state()
            raise
        finally:
            if shuffle is not None:
                shuffle.join()

        # the one host sync of the update: device state and per-mini-batch trace, two async copies, one wait
        self._state_host.copy_(self.device_state, non_blocking=True)
        engine.trace_host.copy_(engine.trace, non_blocking=True)
        engine.read_status()
        torch.cuda.current_stream(self.device).synchronize()
        failure = engine.failure()
        if failure is not None:
            self._restore_state()
            engine.clear_status()
            raise RuntimeError(f"{failure}; the update was rolled back (parameters, optimiser state and normaliser "
                               "statistics are those before it, the rollout is kept)")
        self._opt_steps += steps
        state = ops.device_state_from_host(self._state_host)
        self.learning_rate = state.learning_rate
        for group in self.optimizer.param_groups:
            group["lr"] = self.learning_rate
        self._sync_optimizer_state()
        n = self.num_learning_epochs * self.num_mini_batches
        self._trace_rows = engine.trace_host.view(-1, 5)[:n].clone()
        st.clear()
        return {"value": state.sum_value_loss / n, "surrogate": state.sum_surrogate_loss / n,
                "entropy": state.sum_entropy / n}

    def _save_state(self) -> None:
        """Device copies of what an update changes, into buffers kept from update to update: the flat parameters and
        Adam moments, and the observation normalisers' statistics (a few MB, copied on the update's stream), plus
        each normaliser's host-side sample count."""
        f = self.flat
        norms = [m.obs_normalizer for m in (self.actor, self.critic) if m.obs_normalization]
        saved = self._saved
        if saved is None or saved["flat"][0].numel() != f.param.numel() or \
                [id(n) for n, _, _ in saved["norms"]] != [id(n) for n in norms]:
            saved = self._saved = {
                "flat": [torch.empty_like(t) for t in (f.param, f.exp_avg, f.exp_avg_sq)],
                "norms": [(n, {k: torch.empty_like(v) for k, v in n.state_dict().items()}, [0]) for n in norms]}
        with torch.no_grad():  # (grouped copies: fewer launches and less host time ahead of the first gather)
            dsts, srcs = list(saved["flat"]), [f.param, f.exp_avg, f.exp_avg_sq]
            for norm, bufs, host_count in saved["norms"]:
                for k, v in bufs.items():
                    dsts.append(v)
                    srcs.append(getattr(norm, k))
                host_count[0] = norm._host_count
            torch._foreach_copy_(dsts, srcs)

    def _restore_state(self) -> None:
        f = self.flat
        saved = self._saved
        with torch.no_grad():
            for dst, src in zip((f.param, f.exp_avg, f.exp_avg_sq), saved["flat"]):
                dst.copy_(src)
            for norm, bufs, host_count in saved["norms"]:
                for k, v in bufs.items():
                    getattr(norm, k).copy_(v)
                norm._host_count = host_count[0]

    @property
    def last_trace(self) -> list[dict]:
        """Per mini-batch of the last update: KL mean, learning rate after the adaptive rule, and the three losses."""
        if self._trace_rows is None:
            return []
        return [dict(kl_mean=t[0], lr=t[1], surrogate=t[2], value=t[3], entropy=t[4])
                for t in self._trace_rows.tolist()]

    def _state_views(self, p) -> dict:
        """The torch optimiser's per-parameter state tensors as views of the flat buffers the kernels update: Adam /
        AdamW exp_avg and exp_avg_sq, RMSprop square_avg; SGD without momentum keeps none."""
        if self.optim_kind == L.OPTIM_SGD:
            return {}
        if self.optim_kind == L.OPTIM_RMSPROP:
            return {"square_avg": self.flat.exp_avg_view(p)}
        return {"exp_avg": self.flat.exp_avg_view(p), "exp_avg_sq": self.flat.exp_avg_sq_view(p)}

    def _sync_optimizer_state(self) -> None:
        """Expose the flat optimiser state through the torch optimiser's state (views, no copies).  Every parameter
        takes the same number of steps, so they share one step tensor, updated in place."""
        if self.optim_kind == L.OPTIM_SGD:
            return
        steps = float(self._opt_steps)
        # a parameter that takes no gradient (learn_std=False) has no optimiser state, as in torch's optimisers, whose
        # step skips parameters whose .grad is None
        learned = [p for p in self.flat.params if p.requires_grad]
        if self._step_tensor is not None and all(
                self.optimizer.state[p].get("step") is self._step_tensor for p in learned):
            self._step_tensor.fill_(steps)
            return
        self._step_tensor = torch.tensor(steps)
        for p in learned:
            s = self.optimizer.state[p]
            s["step"] = self._step_tensor
            s.update(self._state_views(p))

    # -- bookkeeping -------------------------------------------------------------------------------------------------
    def train_mode(self) -> None:
        self.actor.train()
        self.critic.train()

    def eval_mode(self) -> None:
        self.actor.eval()
        self.critic.eval()

    def save(self) -> dict:
        """ppo.py:374-385."""
        return {"actor_state_dict": self._raw_actor.state_dict(), "critic_state_dict": self._raw_critic.state_dict(),
                "optimizer_state_dict": self.optimizer.state_dict()}

    def load(self, loaded_dict: dict, load_cfg: dict | None, strict: bool) -> bool:
        """ppo.py:387-411.  Loaded Adam moments are copied into the flat buffers the kernels update."""
        if load_cfg is None:
            load_cfg = {"actor": True, "critic": True, "optimizer": True, "iteration": True, "rnd": True}
        if load_cfg.get("actor"):
            self._raw_actor.load_state_dict(loaded_dict["actor_state_dict"], strict=strict)
        if load_cfg.get("critic"):
            self._raw_critic.load_state_dict(loaded_dict["critic_state_dict"], strict=strict)
        if load_cfg.get("optimizer"):
            self.optimizer.load_state_dict(loaded_dict["optimizer_state_dict"])
            self.learning_rate = self.optimizer.param_groups[0]["lr"]
            steps = 0
            with torch.no_grad():
                for p in self.flat.params:
                    s = self.optimizer.state.get(p, {})
                    views = self._state_views(p)
                    self.flat.exp_avg_view(p).zero_()
                    self.flat.exp_avg_sq_view(p).zero_()
                    if views and all(k in s for k in views):
                        for k, v in views.items():
                            v.copy_(s[k])
                        steps = max(steps, int(float(s["step"])))
            self._opt_steps = steps
            if steps > 0:
                self._sync_optimizer_state()
        return load_cfg.get("iteration", False)

    def get_policy(self) -> MLPModel:
        return self._raw_actor

    def compile(self, mode: str | None = None) -> None:
        """Upstream wraps the models in torch.compile; the HIP path has its own kernels, so only None is accepted."""
        if mode is not None:
            raise NotImplementedError("torch_compile_mode is not applicable to the HIP PPO path")

    def broadcast_parameters(self) -> None:
        raise NotImplementedError("multi-GPU training is not implemented by the HIP PPO plugin")

    def reduce_parameters(self) -> None:
        raise NotImplementedError("multi-GPU training is not implemented by the HIP PPO plugin")

    @staticmethod
    def construct_algorithm(obs: Mapping, env, cfg: dict, device: str) -> "PPO":
        """ppo.py:428-465 (actor then critic construction consumes the global RNG in upstream's order)."""
        alg_class, alg_cfg = resolve_class(cfg["algorithm"])
        actor_class, actor_cfg = resolve_class(cfg["actor"])
        critic_class, critic_cfg = resolve_class(cfg["critic"])
        if alg_cfg.get("rnd_cfg"):
            raise NotImplementedError("RND is not on the HIP PPO path")
        cfg["obs_groups"] = resolve_obs_groups(obs, cfg.get("obs_groups", {}), ["actor", "critic"])
        alg_cfg.pop("share_cnn_encoders", None)
        actor = actor_class(obs, cfg["obs_groups"], "actor", env.num_actions, **actor_cfg)
        critic = critic_class(obs, cfg["obs_groups"], "critic", 1, **critic_cfg)
        storage = RolloutStorage("rl", env.num_envs, cfg["num_steps_per_env"], obs, [env.num_actions], device)
        alg = alg_class(actor, critic, storage, device=device, **alg_cfg, multi_gpu_cfg=cfg.get("multi_gpu"))
        alg.compile(cfg.get("torch_compile_mode"))
        return alg


HipPPO = PPO
