"""The rollout side on the GPU against the CPU oracle: ``act`` / ``process_env_step`` / ``compute_returns``
(upstream rsl_rl/algorithms/ppo.py:124-191) with feed-forward and with LSTM actor and critic (rsl_rl/modules/rnn.py:35-71,
rsl_rl/storage/rollout_storage.py:333-359).

Same initial weights; each step both sides see the same observations, rewards, dones and time-outs (drawn from a
generator of their own).  Each side runs its rollout after the same torch.manual_seed: the plugin draws its action
noise from torch's CPU generator exactly as upstream's torch.normal(mean, std) does, so the actions themselves are
compared, with the policy mean and std, the values and log-probabilities, the LSTM states the models carry (zeroed for
done envs) and the states the storage saves before each step, the stored rewards and GAE.  Bar: 1e-5 relative (fp32
GEMMs of a different summation order over a few steps)."""

from __future__ import annotations

import torch

import pytest

from oracle import rollout as R
from tests.parity import make_hip, rel_err

pytestmark = pytest.mark.gpu


def _workload(layers: int = 1, rnn_type: str = "lstm"):
    w = R.scaled(R.WORKLOADS["lstm256"], num_envs=96, steps=6, hidden_dims=[64, 32])
    w["rnn"] = dict(w["rnn"], rnn_hidden_dim=64, rnn_num_layers=layers, rnn_type=rnn_type)
    w["obs_normalization"] = True
    return w


def _env_inputs(w: dict, seed: int, time_outs: bool = False) -> list[dict]:
    """Observations, rewards, dones (and time-outs) of every step, from a generator of their own (the global CPU
    generator stays the policy's)."""
    g = torch.Generator().manual_seed(seed)
    n = w["num_envs"]

    def obs():
        out = {}
        for name, (kind, width) in w["obs"].items():
            out[name] = torch.randn(n, width, generator=g) if kind == "normal" else \
                torch.rand(n, width, generator=g) * 2.0 - 1.0
        return out

    steps = [{"obs": obs()}]
    for _ in range(w["steps"]):
        d = {"rewards": 0.1 * torch.randn(n, generator=g), "dones": (torch.rand(n, generator=g) < 0.2).float()}
        if time_outs:
            d["time_outs"] = d["dones"] * (torch.rand(n, generator=g) < 0.5).float()
        d["obs"] = obs()
        steps.append(d)
    return steps


def _states(h) -> tuple:
    """A recurrent model's state as a tuple: (h, c) for the LSTM, (h,) for the GRU."""
    return h if isinstance(h, tuple) else (h,)


def _rollout(alg, env: list[dict], dev, seed: int) -> list[dict]:
    """One rollout of alg on the recorded env inputs after torch.manual_seed(seed); per step the transition's
    tensors (on the CPU) and the models' carried states after the step."""
    torch.manual_seed(seed)
    to = (lambda d: {k: v.to(dev) for k, v in d.items()}) if dev is not None else (lambda d: d)
    rec = []
    with torch.inference_mode():
        for step in range(len(env) - 1):
            alg.act(to(env[step]["obs"]))
            tr = alg.transition
            r = {"actions": tr.actions.cpu().clone(), "values": tr.values.cpu().clone(),
                 "logp": tr.actions_log_prob.cpu().clone(),
                 "params": [p.cpu().clone() for p in tr.distribution_params],
                 "hidden": [None if h is None else [x.cpu().clone() for x in _states(h)] for h in tr.hidden_states]}
            e = env[step + 1]
            extras = {"time_outs": e["time_outs"].to(dev) if dev is not None else e["time_outs"]} \
                if "time_outs" in e else {}
            alg.process_env_step(to(e["obs"]), e["rewards"].to(dev) if dev is not None else e["rewards"],
                                 e["dones"].to(dev) if dev is not None else e["dones"], extras)
            r["carried"] = [None if m.get_hidden_state() is None else
                            [x.cpu().clone() for x in _states(m.get_hidden_state())] for m in (alg.actor, alg.critic)]
            rec.append(r)
    r_state = torch.get_rng_state()
    return rec, r_state


@pytest.mark.parametrize("rnn_type,layers", [("lstm", 1), ("lstm", 2), ("gru", 1), ("gru", 2)])
def test_recurrent_rollout_matches_oracle(rnn_type, layers):
    w = _workload(layers, rnn_type)
    states = 2 if rnn_type == "lstm" else 1
    ora = R.make_oracle(w, seed=0)
    ora.train_mode()
    hip = make_hip(w, seed=0)
    with torch.no_grad():
        hip.actor.load_state_dict(ora.actor.state_dict())
        hip.critic.load_state_dict(ora.critic.state_dict())
    dev = hip.device
    n = w["num_envs"]
    env = _env_inputs(w, 11)
    rh, st_h = _rollout(hip, env, dev, seed=21)
    ro, st_o = _rollout(ora, env, None, seed=21)
    assert torch.equal(st_h, st_o), "the rollout must take upstream's draws from the CPU generator"
    for step, (a, b) in enumerate(zip(rh, ro)):
        assert rel_err(a["actions"], b["actions"]) < 1e-5, step
        assert rel_err(a["params"][0], b["params"][0]) < 1e-5, step
        assert rel_err(a["values"], b["values"]) < 1e-5, step
        assert rel_err(a["logp"], b["logp"]) < 1e-5, step
        for side in (0, 1):
            sh, so = a["hidden"][side], b["hidden"][side]
            if step == 0:
                assert sh is None and so is None
                continue
            assert len(sh) == len(so) == states
            for x, y in zip(sh, so):
                assert x.shape == y.shape == (layers, n, w["rnn"]["rnn_hidden_dim"])
                assert rel_err(x, y) < 1e-5, (step, side)
        dones = env[step + 1]["dones"]
        for x, y in zip(a["carried"], b["carried"]):
            for xs, ys in zip(x, y):
                assert torch.equal(xs[:, dones == 1], torch.zeros_like(ys[:, dones == 1]))
                assert rel_err(xs, ys) < 1e-5, step
    with torch.inference_mode():
        # the stored states: step 0 stays zero (no state yet), later steps the state before that step
        for side in ("a", "c"):
            for a, b in zip(getattr(hip.storage, f"saved_hidden_state_{side}"),
                            getattr(ora.storage, f"saved_hidden_state_{side}")):
                assert a.shape == b.shape
                assert rel_err(a, b) < 1e-5
        # the bootstrap forward leaves the critic's rollout state as it was
        obs = env[-1]["obs"]
        before = [t.clone() for t in _states(hip.critic.get_hidden_state())]
        hip.compute_returns({k: v.to(dev) for k, v in obs.items()})
        ora.compute_returns(obs)
        for a, b in zip(_states(hip.critic.get_hidden_state()), before):
            assert torch.equal(a, b)
        assert rel_err(hip.storage.returns, ora.storage.returns) < 1e-5


def test_mlp_rollout_matches_oracle():
    """The feed-forward rollout side: humanoid-shaped actor / critic (separate observation groups, observation
    normalisation) over several steps with dones and time-outs.  Per step: the actions (the same CPU-generator noise
    scaled by the GPU's std and added to its mean), the policy mean and std, the values and the stored
    log-probabilities; then the stored rewards (time-out bootstrap r + gamma V(s_t) on time-outs, ppo.py:150-156) and
    the returns / advantages of compute_returns.  Bar: 1e-5 relative."""
    w = R.scaled(R.WORKLOADS["humanoid"], num_envs=96, steps=5, hidden_dims=[64, 32])
    ora = R.make_oracle(w, seed=0)
    ora.train_mode()
    hip = make_hip(w, seed=0)
    with torch.no_grad():
        hip.actor.load_state_dict(ora.actor.state_dict())
        hip.critic.load_state_dict(ora.critic.state_dict())
    dev = hip.device
    env = _env_inputs(w, 5, time_outs=True)
    rh, st_h = _rollout(hip, env, dev, seed=9)
    ro, st_o = _rollout(ora, env, None, seed=9)
    assert torch.equal(st_h, st_o), "the rollout must take upstream's draws from the CPU generator"
    for step, (a, b) in enumerate(zip(rh, ro)):
        assert rel_err(a["actions"], b["actions"]) < 1e-5, step
        for x, y in zip(a["params"], b["params"]):
            assert rel_err(x, y) < 1e-5, step
        assert rel_err(a["values"], b["values"]) < 1e-5, step
        assert rel_err(a["logp"], b["logp"]) < 1e-5, step
    with torch.inference_mode():
        assert rel_err(hip.storage.rewards, ora.storage.rewards) < 1e-5
        assert torch.equal(hip.storage.dones.cpu().float(), ora.storage.dones.float())
        obs = env[-1]["obs"]
        hip.compute_returns({k: v.to(dev) for k, v in obs.items()})
        ora.compute_returns(obs)
        assert rel_err(hip.storage.returns, ora.storage.returns) < 1e-5
        assert rel_err(hip.storage.advantages, ora.storage.advantages) < 1e-5


@pytest.mark.parametrize("recurrent", [False, True])
def test_learn_iterations_follow_upstreams_random_stream(recurrent):
    """Two learn iterations (rollout -> compute_returns -> update, twice), upstream's runner loop
    (rsl_rl/runners/on_policy_runner.py:95-112), on both sides after the same seed: the CPU generator is at the same
    position after every rollout and every update, so the second rollout's actions and the second update's mini-batch
    indices are upstream's too (bit-identical indices, actions to 1e-5), and the learning-rate decisions agree."""
    if recurrent:
        w = _workload()
    else:
        w = R.scaled(R.WORKLOADS["humanoid"], num_envs=128, steps=8, hidden_dims=[64, 32])
    ora = R.make_oracle(w, seed=0)
    ora.train_mode()
    hip = make_hip(w, seed=0)
    with torch.no_grad():
        hip.actor.load_state_dict(ora.actor.state_dict())
        hip.critic.load_state_dict(ora.critic.state_dict())
    dev = hip.device
    envs = [_env_inputs(w, 100 + it) for it in range(2)]

    def learn(alg, device):
        out = []
        torch.manual_seed(42)
        for env in envs:
            rec, st_roll = _rollout_no_seed(alg, env, device)
            with torch.inference_mode():
                obs = env[-1]["obs"]
                alg.compute_returns({k: v.to(device) for k, v in obs.items()} if device is not None else obs)
            alg.update()
            lr_trace = [t["lr"] for t in (alg.last_trace if device is not None else alg.trace)]
            perm = None
            if not recurrent:
                perm = hip._perm_host.clone() if device is not None else \
                    torch.cat([t["indices"] for t in alg.trace[:alg.num_mini_batches]])
            out.append({"rec": rec, "roll_state": st_roll, "update_state": torch.get_rng_state(), "perm": perm,
                        "lr": lr_trace})
        return out

    hs = learn(hip, dev)
    os_ = learn(ora, None)
    for it, (h, o) in enumerate(zip(hs, os_)):
        assert torch.equal(h["roll_state"], o["roll_state"]), it
        assert torch.equal(h["update_state"], o["update_state"]), it
        if not recurrent:
            assert torch.equal(h["perm"], o["perm"]), it
        assert h["lr"] == o["lr"], it
        for step, (a, b) in enumerate(zip(h["rec"], o["rec"])):
            assert rel_err(a["actions"], b["actions"]) < 1e-5, (it, step)


def _rollout_no_seed(alg, env, dev):
    to = (lambda d: {k: v.to(dev) for k, v in d.items()}) if dev is not None else (lambda d: d)
    rec = []
    with torch.inference_mode():
        for step in range(len(env) - 1):
            alg.act(to(env[step]["obs"]))
            rec.append({"actions": alg.transition.actions.cpu().clone()})
            e = env[step + 1]
            alg.process_env_step(to(e["obs"]), e["rewards"].to(dev) if dev is not None else e["rewards"],
                                 e["dones"].to(dev) if dev is not None else e["dones"], {})
    return rec, torch.get_rng_state()
