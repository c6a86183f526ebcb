"""The LSTM and GRU kernels through the C ABI (ppo_lstm_pack / ppo_gru_pack, _seq_fwd / _seq_bwd, _unpack_grads,
plus the input projection and weight gradients through the linear entry points) against an fp64 reference of
torch.nn.LSTM's / torch.nn.GRU's cell equations over the masked per-env sequence (state multiplied by 1 - done after
each step) with autograd gradients.  The
equivalence of that sequence with upstream's padded trajectories is pinned on the CPU
(tests/test_oracle_recurrent.py)."""

from __future__ import annotations

import math

import pytest
import torch

from tests.parity import rel_err

pytestmark = pytest.mark.gpu


def _reference(x, h0, c0, dones, w_ih, w_hh, b_ih, b_hh, dh):
    """fp64: outputs [T, E, H] and d(sum(out * dh))/d(w_ih, w_hh, b_ih, b_hh)."""
    params = [p.detach().double().requires_grad_(True) for p in (w_ih, w_hh, b_ih, b_hh)]
    w_ih, w_hh, b_ih, b_hh = params
    H = h0.shape[1]
    h, c = h0.double(), c0.double()
    outs = []
    for t in range(x.shape[0]):
        g = x[t].double() @ w_ih.t() + b_ih + h @ w_hh.t() + b_hh
        i, f, gg, o = (g[:, k * H:(k + 1) * H] for k in range(4))
        c = torch.sigmoid(f) * c + torch.sigmoid(i) * torch.tanh(gg)
        h = torch.sigmoid(o) * torch.tanh(c)
        outs.append(h)
        keep = (1.0 - dones[t].double())[:, None]
        h, c = h * keep, c * keep
    out = torch.stack(outs)
    (out * dh.double()).sum().backward()
    return out.detach(), [p.grad for p in params]


@pytest.mark.parametrize("one_launch", [False, True], ids=["per_step", "one_launch"])
@pytest.mark.parametrize("T,E,D,H", [(7, 64, 48, 256), (5, 200, 13, 8), (24, 1024, 48, 256), (6, 100, 20, 96),
                                     (4, 1000, 16, 128), (9, 130, 7, 32)])
def test_lstm_sequence_forward_and_backward(cuda, T, E, D, H, one_launch):
    """Both the per-step launches and the whole-sequence launches (H = 8 takes the per-step path either way)."""
    from tt_rsl_rl_amd import ops

    torch.manual_seed(T * 1000 + H)
    lstm = torch.nn.LSTM(D, H)
    w_ih, w_hh, b_ih, b_hh = (p.detach() for p in (lstm.weight_ih_l0, lstm.weight_hh_l0, lstm.bias_ih_l0,
                                                    lstm.bias_hh_l0))
    x = torch.randn(T, E, D)
    h0, c0 = torch.randn(E, H) * 0.5, torch.randn(E, H) * 0.5
    dones = (torch.rand(T, E) < 0.2).float()
    dh = torch.randn(T, E, H) / math.sqrt(H)
    ref_out, ref_grads = _reference(x, h0, c0, dones, w_ih, w_hh, b_ih, b_hh, dh)

    dev = cuda
    g = lambda t: t.contiguous().to(dev)
    pk = ops.LstmPacked(D, H, dev)
    wd = [g(w) for w in (w_ih, w_hh, b_ih, b_hh)]
    ops.lstm_pack([(*wd, pk)])
    R = T * E
    xf = g(x.reshape(R, D))
    gx = torch.empty(R, 4 * H, device=dev)
    ops.linear_fwd([(xf, pk.w_ih_g, pk.b_g, gx, None)], R, elu=False)
    keep = g(1.0 - dones.reshape(R))
    q = dict(packed=pk, hidden=H, gx=gx, h0=g(h0), c0=g(c0), keep=keep, h=torch.empty(R, H, device=dev),
             hs=torch.empty(R + E, H, device=dev), c=torch.empty(R, H, device=dev),
             gates=torch.empty(R, 4 * H, device=dev), dh=g(dh.reshape(R, H)),
             dgates=torch.empty(R, 4 * H, device=dev), dc=torch.empty(E, H, device=dev))
    sync = torch.zeros(ops.lstm_seq_sync_words(1, E), dtype=torch.int32, device=dev) if one_launch else None
    ops.lstm_seq_fwd([q], T, E, sync)
    assert rel_err(q["h"].view(T, E, H), ref_out) < 1e-5
    ops.lstm_seq_bwd([q], T, E, sync)
    dw_ih_g, dw_hh_g = torch.empty(4 * H, D, device=dev), torch.empty(4 * H, H, device=dev)
    db_g, db_g2 = torch.empty(4 * H, device=dev), torch.empty(4 * H, device=dev)
    ops.linear_bwd_dw([(q["dgates"], q["hs"][:R], dw_hh_g, db_g), (q["dgates"], xf, dw_ih_g, db_g2)], R)
    grads = [torch.empty_like(t) for t in wd]
    ops.lstm_unpack_grads([(dw_ih_g, dw_hh_g, db_g, *grads)])
    torch.cuda.synchronize()
    for name, got, want in zip(("w_ih", "w_hh", "b_ih", "b_hh"), grads, ref_grads):
        assert rel_err(got, want) < 1e-5, name
    assert torch.equal(db_g, db_g2)  # the same column sums of dgates, in the same fixed order
    if sync is not None:
        assert int(sync[0]) == 0


def _reference_gru(x, h0, dones, w_ih, w_hh, b_ih, b_hh, dh):
    """fp64 over torch.nn.GRU's cell equations (gates r, z, n; n = tanh(W_in x + b_in + r (W_hn h + b_hn)),
    h' = (1 - z) n + z h): outputs [T, E, H] and d(sum(out * dh))/d(w_ih, w_hh, b_ih, b_hh)."""
    params = [p.detach().double().requires_grad_(True) for p in (w_ih, w_hh, b_ih, b_hh)]
    w_ih, w_hh, b_ih, b_hh = params
    H = h0.shape[1]
    h = h0.double()
    outs = []
    for t in range(x.shape[0]):
        gi = x[t].double() @ w_ih.t() + b_ih
        gh = h @ w_hh.t() + b_hh
        r = torch.sigmoid(gi[:, :H] + gh[:, :H])
        z = torch.sigmoid(gi[:, H:2 * H] + gh[:, H:2 * H])
        n = torch.tanh(gi[:, 2 * H:] + r * gh[:, 2 * H:])
        h = (1.0 - z) * n + z * h
        outs.append(h)
        h = h * (1.0 - dones[t].double())[:, None]
    out = torch.stack(outs)
    (out * dh.double()).sum().backward()
    return out.detach(), [p.grad for p in params]


@pytest.mark.parametrize("one_launch", [False, True], ids=["per_step", "one_launch"])
@pytest.mark.parametrize("T,E,D,H", [(7, 64, 48, 256), (5, 200, 13, 8), (24, 1024, 48, 256), (6, 100, 20, 96),
                                     (9, 130, 7, 32)])
def test_gru_sequence_forward_and_backward(cuda, T, E, D, H, one_launch):
    """The GRU on the LSTM's kernels (ppo_gru_pack's four-slot layout, cell = PPO_CELL_GRU, ppo_gru_unpack_grads)
    against nn.GRU's equations in fp64 with autograd gradients; per-step and whole-sequence launches."""
    from tt_rsl_rl_amd import ops

    torch.manual_seed(T * 1000 + H + 7)
    gru = torch.nn.GRU(D, H)
    w_ih, w_hh, b_ih, b_hh = (p.detach() for p in (gru.weight_ih_l0, gru.weight_hh_l0, gru.bias_ih_l0,
                                                    gru.bias_hh_l0))
    # biases of the size the weights have, so a bias mapped to the wrong slot shows
    b_ih, b_hh = torch.randn_like(b_ih) * 0.3, torch.randn_like(b_hh) * 0.3
    x = torch.randn(T, E, D)
    h0 = torch.randn(E, H) * 0.5
    dones = (torch.rand(T, E) < 0.2).float()
    dh = torch.randn(T, E, H) / math.sqrt(H)
    ref_out, ref_grads = _reference_gru(x, h0, dones, w_ih, w_hh, b_ih, b_hh, dh)

    dev = cuda
    g = lambda t: t.contiguous().to(dev)
    pk = ops.LstmPacked(D, H, dev)
    wd = [g(w) for w in (w_ih, w_hh, b_ih, b_hh)]
    ops.lstm_pack([(*wd, pk)], gru=True)
    R = T * E
    xf = g(x.reshape(R, D))
    gx = torch.empty(R, 4 * H, device=dev)
    ops.linear_fwd([(xf, pk.w_ih_g, pk.b_g, gx, None)], R, elu=False)
    keep = g(1.0 - dones.reshape(R))
    h0d = g(h0)
    q = dict(packed=pk, hidden=H, gx=gx, h0=h0d, c0=h0d, keep=keep, h=torch.empty(R, H, device=dev),
             hs=torch.empty(R + E, H, device=dev), c=torch.empty(R, H, device=dev),
             gates=torch.empty(R, 4 * H, device=dev), dh=g(dh.reshape(R, H)),
             dgates=torch.empty(R, 4 * H, device=dev), dc=torch.empty(E, H, device=dev), gru=True)
    sync = torch.zeros(ops.lstm_seq_sync_words(1, E), dtype=torch.int32, device=dev) if one_launch else None
    ops.lstm_seq_fwd([q], T, E, sync)
    assert rel_err(q["h"].view(T, E, H), ref_out) < 1e-5
    assert torch.equal(q["c"], q["h"])  # the GRU's state is h
    ops.lstm_seq_bwd([q], T, E, sync)
    dw_ih_g, dw_hh_g = torch.empty(4 * H, D, device=dev), torch.empty(4 * H, H, device=dev)
    db_g = torch.empty(4 * H, device=dev)
    ops.linear_bwd_dw([(q["dgates"], q["hs"][:R], dw_hh_g, db_g), (q["dgates"], xf, dw_ih_g, None)], R)
    grads = [torch.empty_like(t) for t in wd]
    ops.lstm_unpack_grads([(dw_ih_g, dw_hh_g, db_g, *grads)], gru=True)
    torch.cuda.synchronize()
    for name, got, want in zip(("w_ih", "w_hh", "b_ih", "b_hh"), grads, ref_grads):
        assert rel_err(got, want) < 1e-5, name
    if sync is not None:
        assert int(sync[0]) == 0


@pytest.mark.parametrize("gru", [False, True], ids=["lstm", "gru"])
@pytest.mark.parametrize("D,H,groups", [(48, 256, (0, 1)), (13, 96, (2, 2)), (7, 8, (3,))])
def test_unpack_grads_norm_adds_the_torch_layout_squares(cuda, D, H, groups, gru):
    """ppo_lstm_unpack_grads_norm / ppo_gru_unpack_grads_norm write the same gradients as the plain unpack (bit for
    bit) and add, per parameter group, the fp64 sum of squares of the torch-layout gradients (both biases of the
    LSTM, the GRU's separate n biases) to the partial rows already there; twice in a row gives the same rows."""
    from tt_rsl_rl_amd import _lib as L, ops

    dev = cuda
    gen = torch.Generator().manual_seed(D * 100 + H + gru)
    G = (3 if gru else 4) * H
    items, plain = [], []
    for _ in groups:
        packed = [torch.randn(4 * H, D, generator=gen).to(dev), torch.randn(4 * H, H, generator=gen).to(dev),
                  torch.randn(4 * H, generator=gen).to(dev)]
        out = [torch.full((G, D), float("nan"), device=dev), torch.full((G, H), float("nan"), device=dev),
               torch.full((G,), float("nan"), device=dev), torch.full((G,), float("nan"), device=dev)]
        ref = [torch.empty_like(t) for t in out]
        items.append((*packed, *out))
        plain.append((*packed, *ref))
    ops.lstm_unpack_grads(plain, gru=gru)
    start = torch.rand(L.DW_NORM_BLOCKS, L.MAX_PARAM_GROUPS, generator=gen, dtype=torch.float64).to(dev)
    runs = []
    for _ in range(2):
        partials = start.clone()
        ops.lstm_unpack_grads(items, gru=gru, norm=(partials, list(groups)))
        runs.append(partials)
    torch.cuda.synchronize()
    for it, ref in zip(items, plain):
        for got, want in zip(it[3:], ref[3:]):
            assert torch.equal(got, want)
    want = start.sum(0).clone()
    for grp, it in zip(groups, items):
        want[grp] += sum(float((t.double() ** 2).sum()) for t in it[3:])
    got = runs[0].sum(0)
    assert torch.allclose(got, want, rtol=1e-12, atol=0), (got, want)
    assert torch.equal(runs[0], runs[1])
    blocks = min(-(-len(groups) * G * (D + H + 1) // 256), L.DW_NORM_BLOCKS)  # (one launch: at most two problems)
    assert torch.equal(runs[0][blocks:], start[blocks:])  # rows past the launch's blocks keep their values


def _random_sequences(dev, T, E, H, count, seed, gru=False):
    from tt_rsl_rl_amd import ops

    gen = torch.Generator().manual_seed(seed)
    G = (3 if gru else 4) * H
    qs = []
    for _ in range(count):
        pk = ops.LstmPacked(8, H, dev)
        w = [torch.randn(G, 8, generator=gen) * 0.3, torch.randn(G, H, generator=gen) / math.sqrt(H),
             torch.randn(G, generator=gen) * 0.1, torch.randn(G, generator=gen) * 0.1]
        ops.lstm_pack([(*(t.to(dev) for t in w), pk)], gru=gru)
        R = T * E
        dones = (torch.rand(R, generator=gen) < 0.05).float()
        h0 = (torch.randn(E, H, generator=gen) * 0.5).to(dev)
        c0 = h0 if gru else (torch.randn(E, H, generator=gen) * 0.5).to(dev)
        qs.append(dict(packed=pk, hidden=H, gx=torch.randn(R, 4 * H, generator=gen).to(dev), h0=h0, c0=c0,
                       keep=(1.0 - dones).to(dev), gru=gru))
    return qs


def _outputs(q, T, E, H, dev):
    R = T * E
    return dict(q, h=torch.full((R, H), float("nan"), device=dev), hs=torch.full((R + E, H), float("nan"), device=dev),
                c=torch.full((R, H), float("nan"), device=dev), gates=torch.full((R, 4 * H), float("nan"), device=dev))


@pytest.mark.parametrize("gru", [False, True], ids=["lstm", "gru"])
@pytest.mark.parametrize("T,E,H,count", [(24, 1024, 256, 2), (9, 200, 64, 1), (5, 70, 96, 2), (4, 8192, 256, 2),
                                         (3, 64, 512, 1), (1, 100, 256, 2), (6, 65, 32, 2)])
def test_one_launch_sequence_matches_per_step_launches(cuda, T, E, H, count, gru):
    """The whole-sequence forward (row groups of 64 envs synchronised through the sync buffer; 8192 envs need more
    row groups than the device holds at once, so blocks take several in turn; H = 512 and T = 1 take the per-step
    launches) gives bit-identical outputs to one launch per step, and leaves the status word clear."""
    from tt_rsl_rl_amd import ops

    dev = cuda
    qs = _random_sequences(dev, T, E, H, count, seed=T * 7919 + E + H, gru=gru)
    per_step = [_outputs(q, T, E, H, dev) for q in qs]
    ops.lstm_seq_fwd(per_step, T, E)
    sync = torch.zeros(ops.lstm_seq_sync_words(count, E), dtype=torch.int32, device=dev)
    for rep in range(2):  # a second call reuses the buffer
        one = [_outputs(q, T, E, H, dev) for q in qs]
        ops.lstm_seq_fwd(one, T, E, sync)
        torch.cuda.synchronize()
        assert int(sync[0]) == 0
        assert int(sync[1]) == 0 and not sync[32::32].any()  # abort word and every row group's counter at zero
        for a, b in zip(per_step, one):
            for k in ("h", "c", "gates"):
                assert torch.equal(a[k], b[k]), (k, rep)
            assert torch.equal(a["hs"], b["hs"]), ("hs", rep)


@pytest.mark.parametrize("gru", [False, True], ids=["lstm", "gru"])
@pytest.mark.parametrize("T,E,H,count", [(24, 1024, 256, 2), (9, 200, 64, 1), (5, 70, 96, 2), (4, 8192, 256, 2),
                                         (3, 64, 512, 1), (6, 65, 32, 2)])
def test_one_launch_backward_matches_per_step_launches(cuda, T, E, H, count, gru):
    """The whole-sequence backward against one launch per step on the same forward: dgates of every step agree to
    fp32 rounding (the recurrent product sums its 4H terms in another order), the status word stays clear, every
    call leaves the row groups' counters at zero (no clearing launch before the backward), and a second call on the
    same buffer gives the same bits."""
    from tt_rsl_rl_amd import ops

    dev = cuda
    qs = _random_sequences(dev, T, E, H, count, seed=T * 31 + E + H, gru=gru)
    gen = torch.Generator().manual_seed(E + H)
    qs = [_outputs(q, T, E, H, dev) for q in qs]
    ops.lstm_seq_fwd(qs, T, E)
    for q in qs:
        q["dh"] = (torch.randn(T * E, H, generator=gen) / math.sqrt(H)).to(dev)
        q["dc"] = torch.empty(E, H, device=dev)
    per_step = [dict(q, dgates=torch.full((T * E, 4 * H), float("nan"), device=dev)) for q in qs]
    ops.lstm_seq_bwd(per_step, T, E)
    sync = torch.zeros(ops.lstm_seq_sync_words(count, E), dtype=torch.int32, device=dev)
    first = None
    for rep in range(2):
        one = [dict(q, dgates=torch.full((T * E, 4 * H), float("nan"), device=dev)) for q in qs]
        ops.lstm_seq_bwd(one, T, E, sync)
        torch.cuda.synchronize()
        assert int(sync[0]) == 0
        assert int(sync[1]) == 0 and not sync[32::32].any()
        for a, b in zip(per_step, one):
            assert torch.isfinite(b["dgates"]).all()
            assert rel_err(b["dgates"], a["dgates"]) < 1e-5, rep
        if first is None:
            first = [b["dgates"].clone() for b in one]
        else:
            assert all(torch.equal(x, b["dgates"]) for x, b in zip(first, one))


def test_sequence_wait_gives_up_and_the_update_raises(cuda):
    """A wait limit of 0 ticks, forced from the host, makes the blocks of a one-launch sequence give up waiting for
    each other: every launch still runs to its end, the sticky status word is set (and stays set through a normal
    call, which clears only the counters), and a recurrent update that hit it raises instead of returning results,
    rolled back to the state before it, after which the next update runs normally."""
    from oracle import rollout as R
    from tests.parity import make_hip
    from tt_rsl_rl_amd import ops

    dev = cuda
    T, E, H = 24, 1024, 256
    qs = [_outputs(q, T, E, H, dev) for q in _random_sequences(dev, T, E, H, 2, seed=5)]
    sync = torch.zeros(ops.lstm_seq_sync_words(2, E), dtype=torch.int32, device=dev)
    ops.lstm_seq_wait_limit(0)
    try:
        ops.lstm_seq_fwd(qs, T, E, sync)
        torch.cuda.synchronize()
    finally:
        assert ops.lstm_seq_wait_limit(None) == 0
    assert int(sync[0]) == 1
    ops.lstm_seq_fwd(qs, T, E, sync)
    torch.cuda.synchronize()
    assert int(sync[0]) == 1
    sync.zero_()
    ops.lstm_seq_fwd(qs, T, E, sync)
    torch.cuda.synchronize()
    assert int(sync[0]) == 0

    w = R.scaled(R.WORKLOADS["lstm256"], num_envs=512, steps=24, hidden_dims=[256, 128])
    hip = make_hip(w, seed=0)
    g = torch.Generator().manual_seed(3)
    st = hip.storage
    for v in st.observations.values():
        v.copy_(torch.randn(v.shape, generator=g))
    st.actions.copy_(torch.randn(st.actions.shape, generator=g))
    st.rewards.copy_(torch.randn(st.rewards.shape, generator=g) * 0.2)
    st.values.copy_(torch.randn(st.values.shape, generator=g))
    mean = torch.randn(st.actions.shape, generator=g)
    st.distribution_params = (mean.to(hip.device), torch.ones_like(st.actions))
    st.actions_log_prob.copy_(torch.distributions.Normal(mean, 1.0).log_prob(st.actions.cpu()).sum(-1, keepdim=True))
    st.step = st.num_transitions_per_env
    hip.compute_returns_from(torch.randn(w["num_envs"], 1, generator=g).to(hip.device))
    before = [t.clone() for t in (hip.flat.param, hip.flat.exp_avg, hip.flat.exp_avg_sq)]
    lr, steps = hip.learning_rate, hip._opt_steps
    ops.lstm_seq_wait_limit(0)
    try:
        with pytest.raises(RuntimeError, match="stopped waiting"):
            hip.update()
    finally:
        ops.lstm_seq_wait_limit(None)
    # the failed update is rolled back: parameters, moments, learning rate and step count as before, status cleared
    for a, b in zip(before, (hip.flat.param, hip.flat.exp_avg, hip.flat.exp_avg_sq)):
        assert torch.equal(a, b)
    assert hip.learning_rate == lr and hip._opt_steps == steps
    assert int(hip._engine.lstm_sync[0]) == 0
    # and the algorithm stays usable: the same update with the normal wait limit completes
    out = hip.update()
    assert all(torch.isfinite(torch.tensor(v)) for v in out.values())
    assert hip._opt_steps == steps + hip.num_learning_epochs * hip.num_mini_batches
    assert not torch.equal(before[0], hip.flat.param)


@pytest.mark.parametrize("T,E,H,D,count,gru,bf16", [
    (24, 1024, 256, 48, 2, False, False), (24, 1024, 256, 48, 2, True, True), (9, 200, 64, 32, 1, False, False),
    (5, 70, 96, 16, 2, False, True), (4, 8192, 256, 48, 2, False, False), (6, 65, 32, 64, 2, True, False),
    (7, 100, 64, 20, 1, False, False), (1, 100, 128, 48, 2, False, False)])
def test_sequence_with_input_projection_matches_the_separate_projection(cuda, T, E, H, D, count, gru, bf16):
    """ppo_lstm_seq_fwd_proj (the input projection done by the sequence call: inside the one-launch sequence for
    inputs of up to 48 columns in 16-column slabs, else as its own launch) gives bit for bit the outputs of
    ppo_linear_fwd(_ex) into gx followed by ppo_lstm_seq_fwd, in the one-launch and the per-step modes, with fp32
    and bf16 operands; x read as a column block of a wider table, as the update reads it.  64 and 20 columns and a
    single step take the separate launch inside the call."""
    from tt_rsl_rl_amd import _lib as L
    from tt_rsl_rl_amd import ops

    dev = cuda
    gen = torch.Generator().manual_seed(T * 13 + E + H + D)
    G = (3 if gru else 4) * H
    R = T * E
    qs, xs = [], []
    for i in range(count):
        pk = ops.LstmPacked(D, H, dev)
        w = [torch.randn(G, D, generator=gen) / math.sqrt(D), torch.randn(G, H, generator=gen) / math.sqrt(H),
             torch.randn(G, generator=gen) * 0.1, torch.randn(G, generator=gen) * 0.1]
        ops.lstm_pack([(*(t.to(dev) for t in w), pk)], gru=gru)
        table = torch.randn(R, 8 + (D + 3) // 4 * 4 + 12, generator=gen).to(dev)
        xs.append(table[:, 8:8 + D])
        dones = (torch.rand(R, generator=gen) < 0.05).float()
        h0 = (torch.randn(E, H, generator=gen) * 0.5).to(dev)
        c0 = h0 if gru else (torch.randn(E, H, generator=gen) * 0.5).to(dev)
        qs.append(dict(packed=pk, hidden=H, gx=torch.full((R, 4 * H), float("nan"), device=dev), h0=h0, c0=c0,
                       keep=(1.0 - dones).to(dev), gru=gru))
    # reference: the projection as its own GEMM launch, then the sequence on gx
    ref = [_outputs(q, T, E, H, dev) for q in qs]
    ops.linear_fwd([(x, q["packed"].w_ih_g, q["packed"].b_g, q["gx"], None) for q, x in zip(ref, xs)], R,
                   act=L.PPO_ACT_NONE, bf16=bf16)
    sync = torch.zeros(ops.lstm_seq_sync_words(count, E), dtype=torch.int32, device=dev)
    ops.lstm_seq_fwd(ref, T, E, sync)
    for mode in ("one_launch", "per_step"):
        got = [_outputs(dict(q, gx=torch.full((R, 4 * H), float("nan"), device=dev)), T, E, H, dev) for q in qs]
        ops.lstm_seq_fwd(got, T, E, sync if mode == "one_launch" else None, proj=xs, bf16=bf16)
        torch.cuda.synchronize()
        assert int(sync[0]) == 0
        for a, b in zip(ref, got):
            for k in ("h", "c", "gates", "hs"):
                assert torch.equal(a[k], b[k]), (mode, k)
