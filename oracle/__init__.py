"""CPU oracle for the PPO update path -- TEST INFRASTRUCTURE ONLY.

This package restates upstream rsl_rl v5.5.2's PPO path (``rsl_rl/algorithms/ppo.py``,
``rsl_rl/storage/rollout_storage.py``, ``rsl_rl/models/mlp_model.py``, ``rsl_rl/models/rnn_model.py``,
``rsl_rl/modules/{mlp,distribution,normalization,rnn}.py``, ``rsl_rl/utils/utils.py``) in plain torch on
the CPU, with ``dict[str, Tensor]`` in place of ``tensordict.TensorDict`` (tensordict is not installed
here, so upstream itself cannot be imported).  It uses the same torch calls in the same order as
upstream, so its results are upstream's results on the same inputs.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import this package,
and only as the checker / baseline.  The product (``tt_rsl_rl_amd``) never imports it.

Pinning (what makes this restatement trustworthy without importing upstream):
  * GAE / advantage normalisation: upstream's hand-computed returns, terminal cut, singleton and
    mean/std tests (tests/algorithms/test_ppo.py:112-259), plus an fp64 brute-force recursion.
  * Mini-batch generator: upstream's coverage / alignment / partition tests
    (tests/storage/test_rollout_storage.py:72-126,371-406,486-491); the permutation is torch.randperm
    on the CPU generator, bit-exact by construction.
  * Gaussian head: closed-form log-prob / entropy / KL tests (tests/modules/test_distribution.py:17-68).
  * Normalizer: tests/modules/test_normalization.py:18-80 and tests/algorithms/test_ppo.py:293-326,
    plus the parallel-moment closed form.
  * Losses / LR rule: the surrogate, value-clip and adaptive-LR tables
    (tests/algorithms/test_ppo.py:385-437) and the Adam first-step test (:492-505).
  * MLP backward, clip_grad_norm_, Adam: torch autograd / torch.nn.utils.clip_grad_norm_ /
    torch.optim.Adam themselves, checked against fp64 finite differences and closed forms in tests.
"""
