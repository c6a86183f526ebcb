"""Oracle pins for the recurrent path (upstream rollout_storage.py:262-331, utils.py:395-463, rnn.py:22-86,
ppo.py:204-233): the recurrent mini-batch generator pairs every trajectory with the hidden state saved at its start
and covers every transition once (upstream tests/storage/test_rollout_storage.py:409-452 restated); a recurrent
mini-batch's surrogate is the per-transition objective (tests/algorithms/test_ppo.py:332-383 restated); and the
padded-trajectory evaluation equals the masked per-env sequence the GPU path computes (state zeroed after a done),
checked in fp64 against a hand-written LSTM cell."""

from __future__ import annotations

import copy

import pytest
import torch

from oracle import ppo_ref as O


def _tagged_storage(num_envs: int, num_steps: int) -> O.RolloutStorage:
    """Every transition carries its flat id (step * num_envs + env) in its fields; hidden states carry
    env + 1000 * step (+20 / +30 for the critic's h / c); dones at (0, env 0) and (T//2, last env)."""
    obs = {"policy": torch.zeros(num_envs, 1)}
    st = O.RolloutStorage(num_envs, num_steps, obs, [1])
    for step in range(num_steps):
        ids = torch.arange(num_envs, dtype=torch.float32) + step * num_envs
        t = O.Transition()
        t.observations = {"policy": ids[:, None]}
        t.actions = ids[:, None]
        t.values = ids[:, None] * 10
        t.actions_log_prob = ids * 20
        t.distribution_params = (ids[:, None] * 30, torch.ones(num_envs, 1))
        t.rewards = ids
        d = torch.zeros(num_envs)
        if step == 0:
            d[0] = 1
        if step == num_steps // 2:
            d[-1] = 1
        t.dones = d
        h = (torch.arange(num_envs, dtype=torch.float32) + 1000 * step)[None, :, None].expand(2, num_envs, 3).clone()
        t.hidden_states = (h, (h + 20, h + 30))
        st.add_transition(t)
    st.returns.copy_(st.values * 10)
    st.advantages.copy_(st.values * 100)
    return st


@pytest.mark.parametrize("num_envs,num_steps,num_batches", [(5, 3, 2), (7, 4, 3), (6, 4, 3)])
def test_trajectory_states_are_the_states_saved_at_episode_starts(num_envs, num_steps, num_batches):
    st = _tagged_storage(num_envs, num_steps)
    batches = list(st.recurrent_mini_batch_generator(num_batches, 1))
    assert sum(b.actions.shape[1] for b in batches) == num_envs
    for b in batches:
        envs = b.actions[0, :, 0].long().tolist()
        starts = []
        for e in envs:
            starts.append(e)  # the state saved at step 0
            starts += [(s + 1) * 1000 + e for s in range(num_steps - 1) if st.dones[s, e, 0]]
        want = torch.tensor(starts, dtype=torch.float32)
        assert torch.equal(b.hidden_states[0][0, :, 0], want)
        assert torch.equal(b.hidden_states[1][0][0, :, 0], want + 20)
        assert torch.equal(b.hidden_states[1][1][0, :, 0], want + 30)
        assert b.masks.sum().item() == num_steps * len(envs)


@pytest.mark.parametrize("num_epochs", [1, 3])
def test_recurrent_batches_are_env_slices_visiting_each_transition_once_per_epoch(num_epochs):
    num_envs, num_steps, m = 7, 4, 3
    st = _tagged_storage(num_envs, num_steps)
    batches = list(st.recurrent_mini_batch_generator(m, num_epochs))
    assert len(batches) == m * num_epochs
    for ep in range(num_epochs):
        ids = torch.cat([b.actions.flatten() for b in batches[ep * m:(ep + 1) * m]]).long().sort().values
        assert torch.equal(ids, torch.arange(num_envs * num_steps))
    # mini-batch i = env slice [i*N/M, (i+1)*N/M), all steps, the same slices every epoch (no shuffling)
    for i, b in enumerate(batches):
        j = i % m
        lo, hi = j * num_envs // m, (j + 1) * num_envs // m
        assert torch.equal(b.actions[:, :, 0], st.actions[:, lo:hi, 0])
        assert torch.equal(b.advantages, st.advantages[:, lo:hi])


def _masked_lstm_fp64(x, h0, c0, dones, w_ih, w_hh, b_ih, b_hh):
    """x [T, E, D]; state [E, H]; dones [T, E]: the cell equations of torch.nn.LSTM (gates i, f, g, o), one
    sequence per env, state multiplied by (1 - done_t) after step t.  Returns the outputs [T, E, H]."""
    H = h0.shape[-1]
    h, c = h0.double(), c0.double()
    outs = []
    for t in range(x.shape[0]):
        gates = x[t].double() @ w_ih.double().t() + b_ih.double() + h @ w_hh.double().t() + b_hh.double()
        i, f, g, o = (gates[:, k * H:(k + 1) * H] for k in range(4))
        c = torch.sigmoid(f) * c + torch.sigmoid(i) * torch.tanh(g)
        h = torch.sigmoid(o) * torch.tanh(c)
        outs.append(h)
        keep = (1.0 - dones[t].double())[:, None]
        h, c = h * keep, c * keep
    return torch.stack(outs)


def _masked_gru_fp64(x, h0, dones, w_ih, w_hh, b_ih, b_hh):
    """The same for torch.nn.GRU's cell equations as its documentation states them (gates r, z, n):
    r = sigma(W_ir x + b_ir + W_hr h + b_hr), z likewise, n = tanh(W_in x + b_in + r (W_hn h + b_hn)),
    h' = (1 - z) n + z h."""
    H = h0.shape[-1]
    h = h0.double()
    outs = []
    for t in range(x.shape[0]):
        gi = x[t].double() @ w_ih.double().t() + b_ih.double()
        gh = h @ w_hh.double().t() + b_hh.double()
        r = torch.sigmoid(gi[:, :H] + gh[:, :H])
        z = torch.sigmoid(gi[:, H:2 * H] + gh[:, H:2 * H])
        n = torch.tanh(gi[:, 2 * H:] + r * gh[:, 2 * H:])
        h = (1.0 - z) * n + z * h
        outs.append(h)
        h = h * (1.0 - dones[t].double())[:, None]
    return torch.stack(outs)


@pytest.mark.parametrize("rnn_type", ["lstm", "gru"])
@pytest.mark.parametrize("num_envs,num_steps,num_batches,layers", [(6, 5, 2, 1), (9, 7, 3, 1), (9, 7, 3, 2),
                                                                   (5, 6, 1, 3)])
def test_padded_trajectories_equal_the_masked_per_env_sequence(num_envs, num_steps, num_batches, layers, rnn_type):
    """The oracle's upstream-style evaluation (split at dones, pad, nn.LSTM / nn.GRU from each trajectory's saved
    start state, unpad) equals one sequence per env from the state saved at step 0 with the state zeroed after every
    done, evaluated with the cell equations written out; with stacked layers, layer by layer, each from its own saved
    state and on the h sequence of the layer below."""
    torch.manual_seed(3)
    D, H = 4, 5
    gru = rnn_type == "gru"
    rnn = O.RNN(D, hidden_dim=H, num_layers=layers, type=rnn_type).double()
    obs = {"policy": torch.zeros(num_envs, D)}
    st = O.RolloutStorage(num_envs, num_steps, obs, [1])
    # a state carried in from a previous rollout (the GRU's: one tensor)
    state = (torch.randn(layers, num_envs, H),) if gru else (torch.randn(layers, num_envs, H),
                                                              torch.randn(layers, num_envs, H))
    for step in range(num_steps):
        t = O.Transition()
        t.observations = {"policy": torch.randn(num_envs, D)}
        t.actions = torch.zeros(num_envs, 1)
        t.values = torch.zeros(num_envs, 1)
        t.actions_log_prob = torch.zeros(num_envs)
        t.distribution_params = (torch.zeros(num_envs, 1), torch.ones(num_envs, 1))
        t.rewards = torch.zeros(num_envs)
        t.dones = (torch.rand(num_envs) < 0.3).float()
        t.hidden_states = (state[0], state[0]) if gru else (state, state)
        st.add_transition(t)
        # what the rollout does: the policy's state after the step (any value), zeroed for done envs
        state = tuple(s.clone().normal_() * (1 - t.dones)[None, :, None] for s in state)
    w = rnn.rnn
    for b, i in zip(st.recurrent_mini_batch_generator(num_batches, 1), range(num_batches)):
        lo, hi = i * num_envs // num_batches, (i + 1) * num_envs // num_batches
        hs = b.hidden_states[0].double() if gru else tuple(s.double() for s in b.hidden_states[0])
        got = rnn(b.observations["policy"].double(), b.masks, hs)
        want = st.observations["policy"][:, lo:hi]
        for k in range(layers):
            h0 = st.saved_hidden_state_a[0][0, k, lo:hi]
            weights = [getattr(w, f"{n}_l{k}") for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")]
            if gru:
                want = _masked_gru_fp64(want, h0, st.dones[:, lo:hi, 0], *weights)
            else:
                c0 = st.saved_hidden_state_a[1][0, k, lo:hi]
                want = _masked_lstm_fp64(want, h0, c0, st.dones[:, lo:hi, 0], *weights)
        assert torch.allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("rnn_type", ["gru", "lstm"])
def test_recurrent_surrogate_is_the_per_transition_objective(rnn_type):
    """One env, 6 steps with a done at step 2, lr 0: update()'s surrogate and its actor gradients equal the
    clipped objective evaluated directly on the recurrent batch."""
    torch.manual_seed(7)

    def make_obs():
        return {"policy": torch.randn(1, 3)}

    obs = make_obs()
    groups = {"actor": ["policy"], "critic": ["policy"]}
    cfg = dict(hidden_dims=[8], rnn_hidden_dim=8, rnn_type=rnn_type)
    actor = O.RNNModel(obs, groups, "actor", 2, distribution_cfg={"class_name": "GaussianDistribution"}, **cfg)
    critic = O.RNNModel(obs, groups, "critic", 1, **cfg)
    st = O.RolloutStorage(1, 6, obs, [2])
    ppo = O.PPO(actor, critic, st, num_learning_epochs=1, num_mini_batches=1, schedule="fixed", learning_rate=0.0,
                value_loss_coef=0.0, entropy_coef=0.0, max_grad_norm=1e6)
    with torch.inference_mode():
        for step in range(6):
            ppo.act(obs)
            obs = make_obs()
            ppo.process_env_step(obs, torch.randn(1), torch.full((1,), float(step == 2)), {})
        ppo.compute_returns(obs)
    ref = copy.deepcopy(actor)
    b = next(st.recurrent_mini_batch_generator(1, 1))
    ref(b.observations, masks=b.masks, hidden_state=b.hidden_states[0], stochastic_output=True)
    logp = torch.distributions.Normal(ref.output_mean, ref.output_std).log_prob(b.actions).sum(-1).flatten()
    ratio = (logp - b.old_actions_log_prob.flatten()).exp()
    adv = b.advantages.flatten().clone()  # a normal tensor (the storage was filled under inference mode)
    want = -torch.minimum(ratio * adv, ratio.clamp(1 - ppo.clip_param, 1 + ppo.clip_param) * adv).mean()
    want.backward()
    losses = ppo.update()
    assert losses["surrogate"] == pytest.approx(want.item(), rel=1e-5, abs=1e-6)
    for p, q in zip(actor.parameters(), ref.parameters()):
        torch.testing.assert_close(p.grad, q.grad)
