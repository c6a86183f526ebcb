"""Host-side logic of the plugin, without a GPU: drop-in construction, initial weights and state_dict layout equal
upstream's (through the oracle), class resolution, rejected options, the packed-table layout and the workload table.
"""

from __future__ import annotations

import copy

import pytest
import torch

from oracle import ppo_ref as O
from oracle import rollout as R
from tt_rsl_rl_amd import workloads as W
from tt_rsl_rl_amd.engine import TableLayout
from tt_rsl_rl_amd.models import MLPModel, RNNModel
from tt_rsl_rl_amd.ppo import PPO, resolve_callable


def test_workload_table_matches_the_oracle_copy():
    assert W.WORKLOADS == R.WORKLOADS
    assert W.ALGORITHM == R.DEFAULT_ALGORITHM


@pytest.mark.parametrize("name", ["flat48", "humanoid", "rough235", "lstm256", "lstm256x3", "gru256", "gru256x2"])
def test_initial_weights_and_state_dict_layout_equal_upstream(name):
    """Same seed -> same default nn.Linear (and nn.LSTM / nn.GRU, of one or several layers) init as upstream (actor
    then critic), same keys, same parameter order."""
    base = name.split("x")[0]
    w = R.scaled(R.WORKLOADS[base.replace("gru", "lstm")], num_envs=8)
    if base.startswith("gru"):
        w["rnn"] = dict(w["rnn"], rnn_type="gru")
    if "x" in name:
        w["rnn"] = dict(w["rnn"], rnn_num_layers=int(name.split("x")[1]))
    ora = R.make_oracle(w, seed=3)
    torch.manual_seed(3)
    cfg = W.train_cfg(w)
    obs = R.zero_obs(w)
    kw = lambda c: {k: v for k, v in c.items() if k != "class_name"}
    cls = RNNModel if "rnn" in w else MLPModel
    actor = cls(obs, cfg["obs_groups"], "actor", w["num_actions"], **kw(cfg["actor"]))
    critic = cls(obs, cfg["obs_groups"], "critic", 1, **kw(cfg["critic"]))
    for mine, ref in ((actor, ora.actor), (critic, ora.critic)):
        sd, rd = mine.state_dict(), ref.state_dict()
        assert list(sd) == list(rd)
        for k in sd:
            assert torch.equal(sd[k], rd[k]), k
        assert [n for n, _ in mine.named_parameters()] == [n for n, _ in ref.named_parameters()]


def test_class_resolution_maps_upstream_names():
    assert resolve_callable("MLPModel") is MLPModel
    assert resolve_callable("rsl_rl.models:MLPModel") is MLPModel
    assert resolve_callable("rsl_rl.algorithms:PPO") is PPO
    assert resolve_callable("tt_rsl_rl_amd.ppo:PPO") is PPO
    assert resolve_callable("RNNModel") is RNNModel
    assert resolve_callable("rsl_rl.models:RNNModel") is RNNModel
    with pytest.raises(ValueError):
        resolve_callable("NoSuchClass")


def _models(w):
    cfg = W.train_cfg(w)
    obs = R.zero_obs(w)
    kw = lambda c: {k: v for k, v in c.items() if k != "class_name"}
    return (MLPModel(obs, cfg["obs_groups"], "actor", w["num_actions"], **kw(cfg["actor"])),
            MLPModel(obs, cfg["obs_groups"], "critic", 1, **kw(cfg["critic"])))


@pytest.mark.parametrize("kwargs, exc", [
    ({"device": "cpu"}, RuntimeError),
    ({"device": "cuda", "rnd_cfg": {"weight": 1.0}}, NotImplementedError),
    ({"device": "cuda", "symmetry_cfg": {"use_data_augmentation": True}}, NotImplementedError),
    ({"device": "cuda", "multi_gpu_cfg": {"global_rank": 0, "world_size": 2}}, NotImplementedError),
    ({"device": "cuda", "optimizer": "lamb"}, ValueError),  # upstream's resolve_optimizer error
    ({"device": "cpu", "use_mixed_precision": True}, RuntimeError),  # (accepted: rejected for the device only)
])
def test_unsupported_options_are_rejected_before_touching_the_gpu(kwargs, exc):
    w = R.scaled(R.WORKLOADS["flat48"], num_envs=8)
    actor, critic = _models(w)
    with pytest.raises(exc):
        PPO(actor, critic, None, **kwargs)


def test_recurrent_options_outside_the_kernels_are_rejected():
    w = R.scaled(R.WORKLOADS["lstm256"], num_envs=8)
    obs, groups = R.zero_obs(w), w["obs_groups"]
    # upstream's rule (rsl_rl/modules/rnn.py:29): "gru" in any case is the GRU, any other name the LSTM
    assert RNNModel(obs, groups, "actor", 12, rnn_type="GRU").rnn.gru
    assert not RNNModel(obs, groups, "actor", 12, rnn_type="rnn").rnn.gru
    with pytest.raises(ValueError, match="rnn_num_layers"):
        RNNModel(obs, groups, "actor", 12, rnn_num_layers=0)
    with pytest.raises(NotImplementedError, match="multiple of 4"):
        RNNModel(obs, groups, "actor", 12, rnn_hidden_dim=30)
    # a recurrent actor with a feed-forward critic
    cfg = W.train_cfg(w)
    kw = lambda c: {k: v for k, v in c.items() if k != "class_name"}
    actor = RNNModel(obs, groups, "actor", 12, **kw(cfg["actor"]))
    critic = MLPModel(obs, groups, "critic", 1, hidden_dims=[8])
    with pytest.raises(NotImplementedError, match="recurrent"):
        PPO(actor, critic, None, device="cuda")


@pytest.mark.parametrize("name", ["elu", "selu", "relu", "crelu", "lrelu", "tanh", "sigmoid", "softplus", "gelu",
                                  "swish", "mish", "identity", "ELU"])
def test_activations_resolve_to_upstream_modules_and_kernel_codes(name):
    """Every activation name upstream resolves (rsl_rl/utils/utils.py:34-68) builds the model with upstream's module in
    every hidden slot and the kernels' code for it; unknown names raise upstream's ValueError."""
    from tt_rsl_rl_amd import _lib as L

    w = R.scaled(R.WORKLOADS["flat48"], num_envs=8)
    cfg = W.train_cfg(w)
    m = MLPModel(R.zero_obs(w), cfg["obs_groups"], "critic", 1, hidden_dims=[8, 4], activation=name)
    ref = O.activation_module(name)
    assert [type(x) for x in m.mlp] == [torch.nn.Linear, type(ref), torch.nn.Linear, type(ref), torch.nn.Linear]
    assert m.act_code == L.ACTIVATIONS[name.lower()]
    with pytest.raises(ValueError, match="Invalid activation"):
        MLPModel(R.zero_obs(w), cfg["obs_groups"], "critic", 1, hidden_dims=[8], activation="swishy")


@pytest.mark.parametrize("da, dc, a", [(96, 99, 29), (48, 48, 12), (235, 235, 12), (3, 5, 1)])
def test_table_layout_is_aligned_and_disjoint(da, dc, a):
    lay = TableLayout(da, dc, a)
    spans = [(lay.xa, da), (lay.xc, dc), (lay.actions, a), (lay.old_mean, a), (lay.old_std, a),
             (lay.old_logp, 1), (lay.adv, 1), (lay.old_values, 1), (lay.returns, 1), (lay.adv_mb, 1)]
    for start, _ in spans[:5]:
        assert start % 4 == 0
    ends = sorted((s, s + n) for s, n in spans)
    for (s0, e0), (s1, e1) in zip(ends, ends[1:]):
        assert e0 <= s1, "columns overlap"
    assert lay.width % 4 == 0 and lay.width >= ends[-1][1]
    rec = TableLayout(da, dc, a, keep=True)
    assert rec.keep >= ends[-1][1] and rec.width % 4 == 0 and rec.width > rec.keep
    if da == dc:  # one latent block for both models
        sh = TableLayout(da, dc, a, shared_obs=True)
        assert sh.xc == sh.xa == 0 and sh.actions == _round4(da) and sh.width == lay.width - _round4(dc)
    else:
        with pytest.raises(ValueError):
            TableLayout(da, dc, a, shared_obs=True)


def _round4(n: int) -> int:
    return (n + 3) // 4 * 4


def test_gemm_flop_counts():
    """Algorithmic FLOPs per update (fwd + input-grad (not for layer 0) + weight-grad, 5 epochs)."""
    assert W.gemm_flops_per_update(W.WORKLOADS["flat48"]) == pytest.approx(1.06791174144e12)
    assert W.gemm_flops_per_update(W.WORKLOADS["humanoid"]) == pytest.approx(1.1739856896e12)
    assert W.gemm_flops_per_update(W.WORKLOADS["rough235"]) == pytest.approx(1.44439246848e12)
    # LSTM 256 on 48 columns, head [256, 128]: 4 728 576 FLOPs per sample-visit over both models, less the
    # recurrent input-grad of each sequence's last step (2 models x 4096 envs x 2*1024*256)
    lstm = W.WORKLOADS["lstm256"]
    assert W.gemm_flops_per_update(lstm) == pytest.approx(5 * (98304 * 4728576 - 2 * 4096 * 524288))


def test_bench_refuses_more_than_one_gpu():
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parent.parent
    res = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert res.returncode != 0 and "ONE GPU" in res.stderr
