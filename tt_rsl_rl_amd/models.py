"""Actor / critic models with upstream rsl_rl's constructor signature, state_dict keys and parameter order.

Mirrors rsl_rl/models/mlp_model.py:19-193, rsl_rl/modules/mlp.py:16-95, rsl_rl/modules/distribution.py:132-238
and rsl_rl/modules/normalization.py:15-84.  Parameters are ordinary ``nn.Parameter`` objects (default
``nn.Linear`` initialisation drawn from the global CPU generator in upstream's order, so a given seed yields
upstream's initial weights); once the PPO plugin binds them they are views into flat device buffers.  The forward
pass on the GPU runs the HIP kernels of libppo_hip.so; CPU tensors are rejected.
"""

from __future__ import annotations

import copy
from typing import Mapping

import numpy as np
import torch
import torch.nn as nn

from . import _lib as L
from . import ops

_ACTIVATIONS = {
    "elu": nn.ELU, "selu": nn.SELU, "relu": nn.ReLU, "crelu": nn.CELU, "lrelu": nn.LeakyReLU, "tanh": nn.Tanh,
    "sigmoid": nn.Sigmoid, "softplus": nn.Softplus, "gelu": nn.GELU, "swish": nn.SiLU, "mish": nn.Mish,
    "identity": nn.Identity,
}


def resolve_nn_activation(name: str) -> nn.Module:
    """rsl_rl/utils/utils.py:34-68."""
    key = name.lower()
    if key not in _ACTIVATIONS:
        raise ValueError(f"Invalid activation function '{name}'. Valid activations are: {list(_ACTIVATIONS)}")
    return _ACTIVATIONS[key]()


def _require_gpu(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{what}: the tt_rsl_rl_amd models run on the GPU through libppo_hip.so only")


class EmpiricalNormalization(nn.Module):
    """rsl_rl/modules/normalization.py:15-84: buffers ``_mean``, ``_var``, ``_std`` [1, D] and ``count``."""

    def __init__(self, shape, eps: float = 1e-2, until: int | None = None) -> None:
        super().__init__()
        self.eps = eps
        self.until = until
        self.register_buffer("_mean", torch.zeros(shape).unsqueeze(0))
        self.register_buffer("_var", torch.ones(shape).unsqueeze(0))
        self.register_buffer("_std", torch.ones(shape).unsqueeze(0))
        self.register_buffer("count", torch.tensor(0, dtype=torch.long))
        self._host_count = 0  # mirror of `count` for the `until` check without a device sync
        self._ws = ops.Workspace()

    @property
    def mean(self) -> torch.Tensor:
        return self._mean.squeeze(0).clone()

    @property
    def std(self) -> torch.Tensor:
        return self._std.squeeze(0).clone()

    def _load_from_state_dict(self, *args, **kwargs):
        super()._load_from_state_dict(*args, **kwargs)
        self._host_count = int(self.count)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _require_gpu(x, "EmpiricalNormalization.forward")
        x = x.contiguous()
        y = torch.empty_like(x)
        ops.obs_normalize(x.view(-1, x.shape[-1]), y.view(-1, x.shape[-1]), self._mean.view(-1), self._std.view(-1),
                          self.eps)
        return y

    def update_columns(self, columns: list[torch.Tensor]) -> None:
        """normalization.py:51-78 on the concatenation of row-major column blocks (no concatenated copy)."""
        if not self.training:
            return
        if self.until is not None and self._host_count >= self.until:
            return
        self._ws.device = columns[0].device
        ops.normalizer_update(columns, self._mean.view(-1), self._var.view(-1), self._std.view(-1), self.count,
                              self._ws)
        self._host_count += columns[0].shape[0]

    def update(self, x: torch.Tensor) -> None:
        _require_gpu(x, "EmpiricalNormalization.update")
        self.update_columns([x.reshape(-1, x.shape[-1])])

    def inverse(self, y: torch.Tensor) -> torch.Tensor:
        return y * (self._std + self.eps) + self._mean


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
        self._mean: torch.Tensor | None = None
        self._std: torch.Tensor | None = None
        self.host_noise = True
        self._host_noise = _HostNoise()

    # parameter in its own space and the clamp bounds that go with it
    @property
    def param(self) -> nn.Parameter:
        return self.std_param if self.std_type == "scalar" else self.log_std_param

    @property
    def kernel_std_type(self) -> int:
        return L.PPO_STD_SCALAR if self.std_type == "scalar" else L.PPO_STD_LOG

    @property
    def param_range(self) -> tuple[float, float]:
        r = self.std_range if self.std_type == "scalar" else self.log_std_range
        return float(r[0]), float(r[1])

    @property
    def input_dim(self) -> int:
        return self.output_dim

    def init_mlp_weights(self, mlp: nn.Module) -> None:
        pass

    def sample_from(self, mean: torch.Tensor, noise: torch.Tensor | None, actions: torch.Tensor,
                    logp: torch.Tensor | None, std_out: torch.Tensor | None) -> None:
        lo, hi = self.param_range
        L.call("ppo_gauss_sample", mean.data_ptr(), mean.stride(0), self.param.data_ptr(), self.kernel_std_type, lo, hi,
               None if noise is None else noise.data_ptr(), 0 if noise is None else noise.stride(0),
               actions.data_ptr(), actions.stride(0), None if logp is None else logp.data_ptr(),
               None if std_out is None else std_out.data_ptr(), 0 if std_out is None else std_out.stride(0),
               mean.shape[0], self.output_dim, torch.cuda.current_stream().cuda_stream)

    def update(self, mean: torch.Tensor) -> None:
        """Record the distribution of the last forward (the std broadcast per row, as upstream's Normal does)."""
        self._mean = mean
        std = torch.empty_like(mean)
        scratch = torch.empty_like(mean)
        self.sample_from(mean, torch.zeros_like(mean), scratch, None, std)
        self._std = std

    def sample(self) -> torch.Tensor:
        """torch.normal(mean, std) (distribution.py:193-195): a standard-normal draw scaled on the GPU.  The draw
        comes from torch's CPU generator (``host_noise``, the default: the stream upstream's CPU run consumes, so the
        actions and every later draw of that stream are upstream's) or from the device's generator."""
        noise = self._host_noise.draw(self._mean.shape, self._mean.device) if self.host_noise \
            else torch.randn_like(self._mean)
        actions = torch.empty_like(self._mean)
        self.sample_from(self._mean, noise, actions, None, None)
        return actions

    @property
    def mean(self) -> torch.Tensor:
        return self._mean

    @property
    def std(self) -> torch.Tensor:
        return self._std

    @property
    def params(self) -> tuple[torch.Tensor, torch.Tensor]:
        return (self._mean, self._std)

    @property
    def entropy(self) -> torch.Tensor:
        # identical for every row: sum_a 0.5 + 0.5 log(2 pi) + log(std_a)
        return (0.5 + 0.5 * np.log(2 * np.pi) + torch.log(self._std)).sum(dim=-1)

    def log_prob(self, outputs: torch.Tensor) -> torch.Tensor:
        outputs = outputs.contiguous()
        logp = torch.empty(outputs.shape[0], device=outputs.device)
        self.sample_from(self._mean, None, outputs.clone(), logp, None)
        return logp

    def deterministic_output(self, mlp_output: torch.Tensor) -> torch.Tensor:
        return mlp_output

    def as_deterministic_output_module(self) -> nn.Module:
        """distribution.py:201-203: the mean is the MLP output itself."""
        return nn.Identity()


class _HostNoise:
    """Standard-normal draws from torch's CPU generator into pinned buffers, copied to the device asynchronously.
    torch.randn(shape) takes exactly the draws torch.normal(mean, std) takes for that shape on the CPU, and
    randn * std + mean (two fp32 roundings, as the kernel evaluates it) is its result.  Two buffer pairs alternate; a
    pinned buffer is refilled only once its previous copy has completed."""

    def __init__(self) -> None:
        self.host: list[torch.Tensor] = []
        self.dev: list[torch.Tensor] = []
        self.done: list = [None, None]
        self.i = 0

    def draw(self, shape, device) -> torch.Tensor:
        shape = tuple(shape)
        if not self.host or tuple(self.host[0].shape) != shape or self.dev[0].device != torch.device(device):
            for ev in self.done:
                if ev is not None:
                    ev.synchronize()
            self.host = [torch.empty(shape, pin_memory=True) for _ in range(2)]
            self.dev = [torch.empty(shape, device=device) for _ in range(2)]
            self.done = [None, None]
        k = self.i
        self.i ^= 1
        if self.done[k] is not None:
            self.done[k].synchronize()
        torch.randn(shape, out=self.host[k])
        self.dev[k].copy_(self.host[k], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self.done[k] = ev
        return self.dev[k]


class _ForwardBuffers:
    """Grow-only activation buffers for rollout-side forwards (no per-call allocation in steady state)."""

    def __init__(self) -> None:
        self.rows = 0
        self.bufs: list[torch.Tensor] = []

    def get(self, rows: int, widths: list[int], device) -> list[torch.Tensor]:
        if rows > self.rows or len(self.bufs) != len(widths) or self.bufs[0].device != torch.device(device):
            cap = max(rows, self.rows)
            self.bufs = [torch.empty(cap, w, device=device) for w in widths]
            self.rows = cap
        return [b[:rows] for b in self.bufs]


class MLPModel(nn.Module):
    """rsl_rl/models/mlp_model.py:19-193 (same signature; registration order normalizer, distribution, mlp)."""

    is_recurrent: bool = False

    def __init__(self, obs: Mapping, obs_groups: dict, obs_set: str, output_dim: int, hidden_dims=(256, 256, 256),
                 activation: str = "elu", obs_normalization: bool = False, distribution_cfg: dict | None = None) -> None:
        super().__init__()
        self.obs_groups, self.obs_dim = self._get_obs_dim(obs, obs_groups, obs_set)
        self.obs_normalization = obs_normalization
        self.obs_normalizer = EmpiricalNormalization(self.obs_dim) if obs_normalization else nn.Identity()
        if distribution_cfg is not None:
            cfg = dict(distribution_cfg)
            name = cfg.pop("class_name")
            short = name.split(":")[-1].split(".")[-1] if isinstance(name, str) else name.__name__
            if short != "GaussianDistribution":
                raise NotImplementedError(f"distribution {name}: only GaussianDistribution is on the HIP path")
            self.distribution: GaussianDistribution | None = GaussianDistribution(output_dim, **cfg)
            mlp_out = self.distribution.input_dim
        else:
            self.distribution = None
            mlp_out = output_dim
        act = resolve_nn_activation(activation)
        self.act_code = L.ACTIVATIONS[activation.lower()]  # the hidden layers' activation in the HIP kernels
        dims = [self._get_latent_dim() if d == -1 else d for d in hidden_dims]
        layers: list[nn.Module] = [nn.Linear(self._get_latent_dim(), dims[0]), act]
        for a, b in zip(dims[:-1], dims[1:]):
            layers += [nn.Linear(a, b), act]
        layers.append(nn.Linear(dims[-1], mlp_out))
        self.mlp = nn.Sequential(*layers)
        self.output_dim = mlp_out
        self._fwd = _ForwardBuffers()

    # -- structure ---------------------------------------------------------------------------------------------------
    def _get_obs_dim(self, obs: Mapping, obs_groups: dict, obs_set: str) -> tuple[list[str], int]:
        groups = list(obs_groups[obs_set])
        dim = 0
        for g in groups:
            if len(obs[g].shape) != 2:
                raise ValueError(f"The MLP model only supports 1D observations, got shape {obs[g].shape} for '{g}'.")
            dim += obs[g].shape[-1]
        return groups, dim

    def _get_latent_dim(self) -> int:
        return self.obs_dim

    @property
    def linears(self) -> list[nn.Linear]:
        return [m for m in self.mlp if isinstance(m, nn.Linear)]

    # -- forward on the GPU ------------------------------------------------------------------------------------------
    def latent_into(self, obs: Mapping, out: torch.Tensor) -> None:
        """Concatenate this model's observation groups into ``out`` [rows, obs_dim], normalised if enabled."""
        col = 0
        norm = self.obs_normalizer if self.obs_normalization else None
        for g in self.obs_groups:
            x = obs[g]
            _require_gpu(x, "MLPModel.forward")
            x = x.reshape(-1, x.shape[-1])
            if x.stride(-1) != 1:
                x = x.contiguous()
            w = x.shape[1]
            dst = out[:, col:col + w]
            if norm is not None:
                ops.obs_normalize(x, dst, norm._mean.view(-1)[col:col + w], norm._std.view(-1)[col:col + w], norm.eps)
            else:
                dst.copy_(x)
            col += w

    def mlp_forward(self, latent: torch.Tensor) -> torch.Tensor:
        rows = latent.shape[0]
        lin = self.linears
        widths = [l.out_features for l in lin[:-1]]
        bufs = self._fwd.get(rows, widths, latent.device)
        x = latent
        for i, l in enumerate(lin[:-1]):
            h = bufs[i]  # hidden layers: only act(z) is needed
            ops.linear_fwd([(x, l.weight, l.bias, None, h)], rows, act=self.act_code)
            x = h
        out = torch.empty(rows, lin[-1].out_features, device=latent.device)
        ops.linear_fwd([(x, lin[-1].weight, lin[-1].bias, out, None)], rows, act=L.PPO_ACT_NONE)
        return out

    def get_latent(self, obs: Mapping, masks=None, hidden_state=None) -> torch.Tensor:
        first = obs[self.obs_groups[0]]
        latent = torch.empty(first.shape[0], self.obs_dim, device=first.device)
        self.latent_into(obs, latent)
        return latent

    def forward(self, obs: Mapping, masks=None, hidden_state=None, stochastic_output: bool = False) -> torch.Tensor:
        if masks is not None:
            raise NotImplementedError("padded (recurrent) batches are not supported by the MLP HIP path")
        out = self.mlp_forward(self.get_latent(obs))
        if self.distribution is not None:
            if stochastic_output:
                self.distribution.update(out)
                return self.distribution.sample()
            return self.distribution.deterministic_output(out)
        return out

    # -- upstream model API ------------------------------------------------------------------------------------------
    def reset(self, dones=None, hidden_state=None) -> None:
        pass

    def get_hidden_state(self):
        return None

    def detach_hidden_state(self, dones=None) -> None:
        pass

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
    def output_distribution_params(self) -> tuple[torch.Tensor, ...]:
        return self.distribution.params

    def get_output_log_prob(self, outputs: torch.Tensor) -> torch.Tensor:
        return self.distribution.log_prob(outputs)

    def get_kl_divergence(self, old_params, new_params) -> torch.Tensor:
        (om, os_), (nm, ns) = old_params, new_params
        r = (os_ / ns).pow(2)
        t1 = ((om - nm) / ns).pow(2)
        return (0.5 * (r + t1 - 1 - r.log())).sum(dim=-1)

    def update_normalization(self, obs: Mapping) -> None:
        if self.obs_normalization and self.obs_groups:
            cols = []
            for g in self.obs_groups:
                x = obs[g]
                cols.append(x.reshape(-1, x.shape[-1]))
            self.obs_normalizer.update_columns(cols)

    def as_jit(self) -> nn.Module:
        """Export copy in plain torch modules (rsl_rl/models/mlp_model.py:163-165, 196-218) -- export, not the hot
        path."""
        return _TorchMLPModel(self)

    def as_onnx(self) -> nn.Module:
        """rsl_rl/models/mlp_model.py:167-169, 221-255."""
        return _OnnxMLPModel(self)

    def to(self, *args, **kwargs):
        """On a GPU device (the one the parameters live on) a no-op that keeps the parameters as views of the
        update's flat buffers.  On any other device a plain-torch inference copy (``TorchPolicy``), which is what
        upstream's ``runner.get_inference_policy(device)`` (rsl_rl/runners/on_policy_runner.py:171-174) then hands
        out; the model itself stays where the update runs."""
        device = torch._C._nn._parse_to(*args, **kwargs)[0]
        if device is not None and torch.device(device).type != "cuda":
            return TorchPolicy(self, device)
        return super().to(*args, **kwargs)

    def cpu(self):
        return self.to("cpu")


class RNN(nn.Module):
    """rsl_rl/modules/rnn.py:22-86 for an LSTM or a GRU of one or more layers, in rollout mode on the GPU.

    As upstream, ``type`` "gru" (any case) selects the GRU and anything else the LSTM.  The parameters carry the torch
    module's names (``rnn.weight_ih_l<k>``, ``rnn.weight_hh_l<k>``, ``rnn.bias_ih_l<k>``, ``rnn.bias_hh_l<k>`` under
    this module, layer after layer) and its initial values: an ``nn.LSTM`` / ``nn.GRU`` is built on the CPU (drawing
    from the global generator exactly as upstream's constructor does) and its tensors are adopted, so no torch RNN
    kernel ever runs.  ``hidden_state`` is upstream's: the LSTM's tuple ``(h, c)``, the GRU's tensor ``h``, each
    [layers, N, H], or None before the first step; every step writes fresh tensors, so a state captured with
    ``get_hidden_state`` stays valid (upstream relies on that in ``compute_returns``).  Layer k > 0 takes layer
    k - 1's new h as its input."""

    def __init__(self, input_size: int, hidden_dim: int = 256, num_layers: int = 1, type: str = "lstm") -> None:
        super().__init__()
        if num_layers < 1:
            raise ValueError(f"rnn_num_layers={num_layers}")
        if hidden_dim % 4 != 0:
            raise NotImplementedError(f"rnn_hidden_dim={hidden_dim}: the HIP recurrent kernels need a multiple of 4")
        self.gru = type.lower() == "gru"
        ref = (nn.GRU if self.gru else nn.LSTM)(input_size=input_size, hidden_size=hidden_dim, num_layers=num_layers)
        self.rnn = nn.Module()
        for k in range(num_layers):
            for name in (f"weight_ih_l{k}", f"weight_hh_l{k}", f"bias_ih_l{k}", f"bias_hh_l{k}"):
                self.rnn.register_parameter(name, nn.Parameter(getattr(ref, name).detach().clone()))
        self.input_size = input_size
        self.hidden_size = hidden_dim
        self.num_layers = num_layers
        self.hidden_state: tuple[torch.Tensor, torch.Tensor] | torch.Tensor | None = None
        self._packed: list[ops.LstmPacked] = []
        self._fwd = _ForwardBuffers()
        self._hs = _ForwardBuffers()
        self._const = _ForwardBuffers()

    def states(self, hidden_state=None) -> tuple:
        """``hidden_state`` (default: the module's) as a tuple of tensors: (h, c) for the LSTM, (h,) for the GRU."""
        hs = self.hidden_state if hidden_state is None else hidden_state
        return hs if isinstance(hs, tuple) else (hs,)

    def layer_input_size(self, k: int) -> int:
        return self.input_size if k == 0 else self.hidden_size

    def layer_weights(self, k: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
        r = self.rnn
        return (getattr(r, f"weight_ih_l{k}"), getattr(r, f"weight_hh_l{k}"), getattr(r, f"bias_ih_l{k}"),
                getattr(r, f"bias_hh_l{k}"))

    @property
    def weights(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
        """Layer 0's weights."""
        return self.layer_weights(0)

    def packed(self, device, k: int = 0) -> ops.LstmPacked:
        """Layer k's gate-interleaved weight copies the kernels read (buffers only; ``ops.lstm_pack`` fills them)."""
        if len(self._packed) != self.num_layers or self._packed[0].w_ih_g.device != torch.device(device):
            self._packed = [ops.LstmPacked(self.layer_input_size(i), self.hidden_size, device)
                            for i in range(self.num_layers)]
        return self._packed[k]

    def forward(self, x: torch.Tensor, masks=None, hidden_state=None) -> torch.Tensor:
        """rnn.py:35-52, rollout mode: one step for every env of ``x`` [N, input_size], layer after layer; returns the
        last layer's h' [N, H]."""
        if masks is not None:
            raise NotImplementedError("padded trajectory batches: the recurrent update evaluates them on the GPU "
                                      "inside PPO.update()")
        _require_gpu(x, "RNN.forward")
        N, H, layers, dev = x.shape[0], self.hidden_size, self.num_layers, x.device
        gx, gates = self._fwd.get(N, [4 * H, 4 * H], dev)
        zero, ones = self._const.get(N, [H, 1], dev)
        ones.fill_(1.0)
        if self.hidden_state is None:
            zero.zero_()
        h_new = torch.empty(layers, N, H, device=dev)
        # the LSTM's new cell state; the GRU's kernels write the state h into this buffer too (unused)
        c_new = torch.empty(layers, N, H, device=dev)
        # hs: the per-step input states the backward reads ([T + 1 blocks of N rows]); unused in rollout mode
        hs = self._hs.get(2 * N, [H], dev)[0]
        inp = x
        for k in range(layers):
            pk = self.packed(dev, k)
            ops.lstm_pack([(*self.layer_weights(k), pk)], gru=self.gru)
            if self.hidden_state is None:
                h0 = c0 = zero
            else:
                st = [s[k].reshape(N, H) for s in self.states()]
                st = [t if t.stride(0) == H else t.contiguous() for t in st]
                h0, c0 = (st[0], st[0]) if self.gru else st
            ops.linear_fwd([(inp, pk.w_ih_g, pk.b_g, gx, None)], N, act=L.PPO_ACT_NONE)
            ops.lstm_seq_fwd([dict(packed=pk, hidden=H, gx=gx, h0=h0, c0=c0, keep=ones.view(-1), h=h_new[k], hs=hs,
                                   c=c_new[k], gates=gates, gru=self.gru)], 1, N)
            inp = h_new[k]
        self.hidden_state = h_new if self.gru else (h_new, c_new)
        return h_new[layers - 1]

    def reset(self, dones: torch.Tensor | None = None, hidden_state=None) -> None:
        """rnn.py:54-71."""
        if dones is None:
            self.hidden_state = hidden_state
        elif self.hidden_state is not None:
            if hidden_state is not None:
                raise NotImplementedError("Resetting the hidden state of done environments with a custom hidden state "
                                          "is not implemented")
            for s in self.states():
                s[..., dones == 1, :] = 0.0

    def detach_hidden_state(self, dones: torch.Tensor | None = None) -> None:
        """rnn.py:73-86: the HIP path keeps no autograd graph, so there is nothing to detach."""


class RNNModel(MLPModel):
    """rsl_rl/models/rnn_model.py:18-107: LSTM or GRU on the (normalised) observations, then the MLP head.

    Registration order as upstream (normaliser, distribution, mlp, then ``rnn``), so the parameter order is
    [distribution, mlp.*, rnn.rnn.weight_ih_l0, weight_hh_l0, bias_ih_l0, bias_hh_l0] and a seed gives upstream's
    initial weights.  Rollout forwards step the recurrent layers on the GPU; the update evaluates whole mini-batches
    of trajectories inside ``PPO.update()``."""

    is_recurrent: bool = True

    def __init__(self, obs: Mapping, obs_groups: dict, obs_set: str, output_dim: int, hidden_dims=(256, 256, 256),
                 activation: str = "elu", obs_normalization: bool = False, distribution_cfg: dict | None = None,
                 rnn_type: str = "lstm", rnn_hidden_dim: int = 256, rnn_num_layers: int = 1) -> None:
        self.latent_dim = rnn_hidden_dim
        super().__init__(obs, obs_groups, obs_set, output_dim, hidden_dims, activation, obs_normalization,
                         distribution_cfg)
        self.rnn = RNN(self.obs_dim, rnn_hidden_dim, rnn_num_layers, rnn_type)

    def _get_latent_dim(self) -> int:
        return self.latent_dim

    def get_latent(self, obs: Mapping, masks=None, hidden_state=None) -> torch.Tensor:
        """rnn_model.py:76-84 in rollout mode."""
        if masks is not None:
            raise NotImplementedError("padded trajectory batches: the recurrent update evaluates them on the GPU "
                                      "inside PPO.update()")
        return self.rnn(super().get_latent(obs))

    def forward(self, obs: Mapping, masks=None, hidden_state=None, stochastic_output: bool = False) -> torch.Tensor:
        out = self.mlp_forward(self.get_latent(obs, masks, hidden_state))
        if self.distribution is not None:
            if stochastic_output:
                self.distribution.update(out)
                return self.distribution.sample()
            return self.distribution.deterministic_output(out)
        return out

    def reset(self, dones=None, hidden_state=None) -> None:
        self.rnn.reset(dones, hidden_state)

    def get_hidden_state(self):
        return self.rnn.hidden_state

    def detach_hidden_state(self, dones=None) -> None:
        self.rnn.detach_hidden_state(dones)

    def as_jit(self) -> nn.Module:
        """Export copy with plain torch modules (rsl_rl/models/rnn_model.py:98-105, 116-175) -- export, not the hot
        path."""
        return _TorchGRUModel(self) if self.rnn.gru else _TorchLSTMModel(self)

    def as_onnx(self) -> nn.Module:
        """rsl_rl/models/rnn_model.py:107-109, 178-247."""
        return _OnnxRNNModel(self)


class _TorchNormalizer(nn.Module):
    """Plain-torch copy of an EmpiricalNormalization for export: the same buffers (``_mean``, ``_var``, ``_std`` [1, D],
    ``count``), forward (x - _mean) / (_std + eps) (rsl_rl/modules/normalization.py:46-48)."""

    def __init__(self, norm: EmpiricalNormalization) -> None:
        super().__init__()
        self.eps = norm.eps
        for name in ("_mean", "_var", "_std", "count"):
            self.register_buffer(name, getattr(norm, name).detach().clone().cpu())

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return (x - self._mean) / (self._std + self.eps)


def _export_parts(model) -> tuple[nn.Module, nn.Module, nn.Module]:
    """CPU copies of the normaliser, the MLP head and the deterministic output (the distribution's mean)."""
    norm = _TorchNormalizer(model.obs_normalizer) if model.obs_normalization else nn.Identity()
    det = model.distribution.as_deterministic_output_module() if model.distribution is not None else nn.Identity()
    return norm, copy.deepcopy(model.mlp).cpu(), det


def _cpu_rnn(model: RNNModel) -> nn.Module:
    """The model's recurrent layers as a CPU nn.GRU / nn.LSTM with its current weights."""
    rnn = model.rnn
    out = (nn.GRU if rnn.gru else nn.LSTM)(rnn.input_size, rnn.hidden_size, num_layers=rnn.num_layers)
    with torch.no_grad():
        for k in range(rnn.num_layers):
            for name, p in zip((f"weight_ih_l{k}", f"weight_hh_l{k}", f"bias_ih_l{k}", f"bias_hh_l{k}"),
                               rnn.layer_weights(k)):
                getattr(out, name).copy_(p.detach().cpu())
    return out


class _TorchMLPModel(nn.Module):
    """TorchScript export copy, rsl_rl/models/mlp_model.py:196-218: normaliser, MLP, deterministic output."""

    def __init__(self, model: MLPModel) -> None:
        super().__init__()
        self.obs_normalizer, self.mlp, self.deterministic_output = _export_parts(model)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = self.obs_normalizer(x)
        out = self.mlp(x)
        return self.deterministic_output(out)

    @torch.jit.export
    def reset(self) -> None:
        pass


class _OnnxMLPModel(nn.Module):
    """ONNX export copy, rsl_rl/models/mlp_model.py:221-255: input "obs", output "actions"."""

    is_recurrent: bool = False

    def __init__(self, model: MLPModel) -> None:
        super().__init__()
        self.obs_normalizer, self.mlp, self.deterministic_output = _export_parts(model)
        self.input_size = model.obs_dim

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = self.obs_normalizer(x)
        out = self.mlp(x)
        return self.deterministic_output(out)

    def get_dummy_inputs(self) -> tuple[torch.Tensor]:
        return (torch.zeros(1, self.input_size),)

    @property
    def input_names(self) -> list[str]:
        return ["obs"]

    @property
    def output_names(self) -> list[str]:
        return ["actions"]


class _TorchLSTMModel(nn.Module):
    """TorchScript export copy, rsl_rl/models/rnn_model.py:147-175: one LSTM step per call on a batch-1 state kept in
    the ``hidden_state`` / ``cell_state`` buffers, ``reset()`` zeroes them."""

    def __init__(self, model: RNNModel) -> None:
        super().__init__()
        norm, mlp, det = _export_parts(model)
        self.obs_normalizer = norm  # upstream's attribute order: normaliser, rnn, mlp, deterministic output
        self.rnn = _cpu_rnn(model)
        self.mlp, self.deterministic_output = mlp, det
        self.register_buffer("hidden_state", torch.zeros(self.rnn.num_layers, 1, self.rnn.hidden_size))
        self.register_buffer("cell_state", torch.zeros(self.rnn.num_layers, 1, self.rnn.hidden_size))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = self.obs_normalizer(x)
        x, (h, c) = self.rnn(x.unsqueeze(0), (self.hidden_state, self.cell_state))
        self.hidden_state[:] = h
        self.cell_state[:] = c
        x = x.squeeze(0)
        out = self.mlp(x)
        return self.deterministic_output(out)

    @torch.jit.export
    def reset(self) -> None:
        self.hidden_state[:] = 0.0
        self.cell_state[:] = 0.0


class _TorchGRUModel(nn.Module):
    """TorchScript export copy, rsl_rl/models/rnn_model.py:116-144: one GRU step per call on a batch-1 state kept in
    the ``hidden_state`` buffer, ``reset()`` zeroes it."""

    def __init__(self, model: RNNModel) -> None:
        super().__init__()
        norm, mlp, det = _export_parts(model)
        self.obs_normalizer = norm
        self.rnn = _cpu_rnn(model)
        self.mlp, self.deterministic_output = mlp, det
        self.register_buffer("hidden_state", torch.zeros(self.rnn.num_layers, 1, self.rnn.hidden_size))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = self.obs_normalizer(x)
        x, h = self.rnn(x.unsqueeze(0), self.hidden_state)
        self.hidden_state[:] = h
        x = x.squeeze(0)
        out = self.mlp(x)
        return self.deterministic_output(out)

    @torch.jit.export
    def reset(self) -> None:
        self.hidden_state[:] = 0.0


class _OnnxRNNModel(nn.Module):
    """ONNX export copy of the recurrent model, rsl_rl/models/rnn_model.py:178-247: the state is an explicit input
    and output (LSTM: inputs "obs", "h_in", "c_in", outputs "actions", "h_out", "c_out"; GRU: without the cell
    state, and None in its output slot)."""

    is_recurrent: bool = True

    def __init__(self, model: RNNModel) -> None:
        super().__init__()
        norm, mlp, det = _export_parts(model)
        self.obs_normalizer = norm
        self.rnn = _cpu_rnn(model)
        self.mlp, self.deterministic_output = mlp, det
        self.rnn_type = "gru" if model.rnn.gru else "lstm"
        self.input_size = model.obs_dim
        self.hidden_size = self.rnn.hidden_size
        self.num_layers = self.rnn.num_layers

    def forward(self, obs: torch.Tensor, h_in: torch.Tensor, c_in: torch.Tensor | None = None):
        x = self.obs_normalizer(obs)
        if self.rnn_type == "lstm":
            x, (h, c) = self.rnn(x.unsqueeze(0), (h_in, c_in))
            x = x.squeeze(0)
            out = self.deterministic_output(self.mlp(x))
            return out, h, c
        x, h = self.rnn(x.unsqueeze(0), h_in)
        x = x.squeeze(0)
        out = self.deterministic_output(self.mlp(x))
        return out, h, None

    def get_dummy_inputs(self) -> tuple[torch.Tensor, ...]:
        obs = torch.zeros(1, self.input_size)
        h_in = torch.zeros(self.num_layers, 1, self.hidden_size)
        if self.rnn_type == "lstm":
            return (obs, h_in, torch.zeros(self.num_layers, 1, self.hidden_size))
        return (obs, h_in)

    @property
    def input_names(self) -> list[str]:
        return ["obs", "h_in", "c_in"] if self.rnn_type == "lstm" else ["obs", "h_in"]

    @property
    def output_names(self) -> list[str]:
        return ["actions", "h_out", "c_out"] if self.rnn_type == "lstm" else ["actions", "h_out"]


class TorchPolicy(nn.Module):
    """Plain-torch inference copy of a plugin model on a device the HIP kernels do not run on (what
    ``model.to("cpu")``, and so upstream's ``runner.get_inference_policy("cpu")``, returns: the plugin model itself
    stays on the GPU, its parameters views of the update's flat buffers).  Upstream's MLPModel / RNNModel forward for
    observation dicts: concatenated groups -> normaliser -> (LSTM / GRU, state carried per env and zeroed by
    ``reset(dones)``) -> MLP -> the distribution's mean.  A copy: later updates do not reach it."""

    def __init__(self, model, device) -> None:
        super().__init__()
        self.obs_groups = list(model.obs_groups)
        self.is_recurrent = bool(model.is_recurrent)
        self.obs_normalizer, self.mlp, self.deterministic_output = _export_parts(model)
        self.rnn = _cpu_rnn(model) if self.is_recurrent else None
        self.hidden_state = None
        self.to(device)

    def forward(self, obs: Mapping, masks=None, hidden_state=None, stochastic_output: bool = False) -> torch.Tensor:
        if stochastic_output or masks is not None:
            raise NotImplementedError("the inference copy evaluates the deterministic policy on rollout observations")
        x = self.obs_normalizer(torch.cat([obs[g] for g in self.obs_groups], dim=-1))
        if self.rnn is not None:
            x, self.hidden_state = self.rnn(x.unsqueeze(0), self.hidden_state)
            x = x.squeeze(0)
        return self.deterministic_output(self.mlp(x))

    def reset(self, dones=None, hidden_state=None) -> None:
        if dones is None:
            self.hidden_state = hidden_state
        elif self.hidden_state is not None:
            states = self.hidden_state if isinstance(self.hidden_state, tuple) else (self.hidden_state,)
            for s in states:
                s[..., dones == 1, :] = 0.0

    def get_hidden_state(self):
        return self.hidden_state
