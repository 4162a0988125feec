"""Speculative-decoding semantics on the CPU: the reference's own unit tests (tests/test_speculative.py:6-44)
restated against the product API and the oracle, the tree flattening, the seeded uniforms (SplitMix64 published
outputs), and the acceptance rule's exact output law (speculative sampling theorem)."""
import random

import numpy as np
import pytest

from oracle import speculative_ref as ref
from seedplane_amd.speculative import (CommitLedger, SpeculativeForest, flatten, uniforms, verify_greedy,
                                       verify_greedy_ids)


def target(prefix):
    # deterministic target of the reference tests: token 1, then 2, then 3, ...
    expected = min(len(prefix), 5)
    logits = [0.0] * 8
    logits[expected] = 1.0
    return logits


@pytest.mark.parametrize('impl', ['product', 'oracle'])
def test_forest_deduplicates_shared_prefix(impl):
    build = SpeculativeForest.build if impl == 'product' else ref.Forest.build
    forest = build([[1, 2, 3], [1, 2, 4], [1, 5]])
    count = forest.node_count if impl == 'product' else forest.node_count()
    assert count == 5 and len(forest.paths) == 3


def test_verifier_accepts_longest_exact_branch_and_corrects_rejection():
    forest = SpeculativeForest.build([[1, 2, 7], [1, 2, 3, 4]])
    result = verify_greedy([0], forest, target)
    assert result.branch == (1, 2, 3, 4) and result.emitted == (1, 2, 3, 4)
    assert result.accepted_draft_tokens == 4 and not result.rejected
    rejected = verify_greedy([0], SpeculativeForest.build([[1, 2, 7]]), target)
    assert rejected.emitted == (1, 2, 3) and rejected.accepted_draft_tokens == 2 and rejected.rejected


def test_commit_ledger_only_advances_on_commit():
    ledger = CommitLedger([0])
    result = verify_greedy(ledger.tokens, SpeculativeForest.build([[1, 2]]), target)
    assert ledger.frontier == 1
    ledger.commit(result)
    assert ledger.tokens == [0, 1, 2] and ledger.frontier == 3 and ledger.commits == 1
    with pytest.raises(ValueError):
        CommitLedger().commit(type(result)((), 0, False, 0, ()))


def test_empty_forest_falls_back_to_target():
    result = verify_greedy([0], SpeculativeForest.build([]), target)
    assert result.emitted == (1,) and result.target_steps == 1


def test_product_verify_matches_oracle_on_random_forests():
    rng = random.Random(0)
    for trial in range(300):
        V = rng.choice([3, 5, 8])
        table = {}

        def logits(prefix):
            if prefix not in table:
                table[prefix] = [rng.choice([0.0, 0.5, 1.0]) for _ in range(V)]   # many ties
            return table[prefix]
        branches = [[rng.randrange(V) for _ in range(rng.randint(0, 4))] for _ in range(rng.randint(0, 5))]
        committed = [rng.randrange(V) for _ in range(rng.randint(1, 3))]
        got = verify_greedy(committed, SpeculativeForest.build(branches), logits)
        exp = ref.verify_greedy(committed, ref.Forest.build(branches), logits)
        assert (got.emitted, got.accepted_draft_tokens, got.rejected, got.target_steps, got.branch) == exp
        ids = verify_greedy_ids(committed, SpeculativeForest.build(branches), lambda p: ref.first_argmax(logits(p)))
        assert ids == got


def test_flatten_layout():
    branches = [[5, 6, 7], [5, 6, 8], [9], [5, 1], [5, 6, 7]]
    t = flatten(42, branches)
    f = SpeculativeForest.build(branches)
    assert t.size == f.node_count + 1 and t.token[0] == 42 and t.parent[0] == -1
    for i in range(1, t.size):
        assert t.parent[i] < i and t.depth[i] == t.depth[t.parent[i]] + 1
    for i in range(t.size):                                        # children contiguous, in first-draw order
        kids = [c for c in range(t.size) if t.parent[c] == i]
        if kids:
            assert kids == list(range(t.first_child[i], t.first_child[i] + t.n_children[i]))
    assert [t.token[c] for c in range(t.first_child[0], t.first_child[0] + t.n_children[0])] == [5, 9]
    n567 = t.node_of_prefix((5, 6, 7))
    assert t.mult[n567] == 2 and t.mult[t.node_of_prefix((5,))] == 4 and t.mult[0] == 5
    # root trials: one per branch in branch order (5, 5, 9, 5, 5 -> node ids of 5 and 9)
    n5, n9 = t.node_of_prefix((5,)), t.node_of_prefix((9,))
    root_trials = t.trials[t.trial_start[0]:t.trial_start[0] + t.n_trials[0]]
    assert root_trials == [n5, n5, n9, n5, n5]
    assert t.ancestors_mask(n567) == (1 << n567) | (1 << t.node_of_prefix((5, 6))) | (1 << t.node_of_prefix((5,))) | 1


def test_splitmix64_published_outputs_and_uniform_stream():
    # SplitMix64 from state 0: the published first outputs
    state, outs = 0, []
    for _ in range(3):
        outs.append(ref.splitmix64(state))
        state = (state + 0x9E3779B97F4A7C15) & ref.MASK64
    assert outs == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    a, b = uniforms(7, 3, 100), ref.uniforms(7, 3, 100)
    assert np.array_equal(a, b) and a.min() >= 0.0 and a.max() < 1.0
    assert not np.array_equal(uniforms(7, 4, 100), a)
    assert abs(float(uniforms(1, 0, 20000).mean()) - 0.5) < 0.01


def test_linear_verify_matches_reference_rollback_rule():
    # benchmark_speculative.py:85-131
    assert ref.linear_verify([3, 4, 5], 9, [4, 5, 6]) == ([9], 0, 0)
    assert ref.linear_verify([3, 4, 5], 3, [4, 7, 6]) == ([3, 4, 7], 2, 2)
    assert ref.linear_verify([3, 4, 5], 3, [4, 5, 6]) == ([3, 4, 5], 3, 3)


@pytest.mark.parametrize('n_branches', [1, 2, 3, 4])
def test_acceptance_law_equals_target_distribution(n_branches):
    # speculative sampling theorem: drafts i.i.d. from q, verified in draw order with the residual rule, emit p
    rng = np.random.default_rng(n_branches)
    for _ in range(5):
        p = rng.dirichlet(np.ones(5) * 0.7)
        q = rng.dirichlet(np.ones(5) * 0.7)
        law = ref.exact_first_token_distribution(p, q, n_branches)
        assert np.abs(law - p).max() < 1e-12


def test_grouping_repeated_drafts_breaks_the_law():
    # trying repeated tokens back to back (instead of in draw order) is not exact from 3 branches on
    rng = np.random.default_rng(3)
    p = rng.dirichlet(np.ones(5) * 0.7)
    q = rng.dirichlet(np.ones(5) * 0.7)
    law = ref.exact_first_token_distribution(p, q, 3, grouped=True)
    assert np.abs(law - p).max() > 1e-4


def test_theorem_check_detects_a_dropped_residual():
    # a planted mistake (retrying children against p instead of the residual) must break the law
    p = np.array([0.5, 0.3, 0.2])
    q = np.array([0.2, 0.2, 0.6])
    good = ref.exact_first_token_distribution(p, q, 2)
    saved = ref._one_level_law

    def no_residual(pp, qq, children):
        out, remaining = np.zeros_like(pp), 1.0
        for x in children:
            a = min(1.0, pp[x] / qq[x])
            out[x] += remaining * a
            remaining *= 1 - a
        return out + remaining * pp
    ref._one_level_law = no_residual
    try:
        bad = ref.exact_first_token_distribution(p, q, 2)
    finally:
        ref._one_level_law = saved
    assert np.abs(good - p).max() < 1e-12 and np.abs(bad - p).max() > 1e-3


def test_oracle_acceptance_walk_samples_the_target_law():
    # Monte Carlo through the uniform-driven oracle walk (the code the GPU kernel is compared with)
    V, nb = 6, 3
    rng = np.random.default_rng(3)
    pl = rng.normal(size=V).astype(np.float32)
    ql = rng.normal(size=V).astype(np.float32)
    p = ref.softmax_weights(pl, 1.0); p /= p.sum()
    q = ref.softmax_weights(ql, 1.0); q /= q.sum()
    counts = np.zeros(V)
    n = 6000
    for s in range(n):
        u = ref.uniforms(11, s, 16)
        drafts = [ref.draw(ref.softmax_weights(ql, 1.0), u[i])[0] for i in range(nb)]
        t = flatten(0, [[d] for d in drafts])
        tree = dict(token=t.token, trial_start=t.trial_start, n_trials=t.n_trials, trials=t.trials)
        P = np.stack([pl] * t.size)
        Q = np.stack([ql] * t.size)
        path, final, used, bonus, _ = ref.accept_tree(P, Q, tree, u[nb:], 1.0, 1)
        first = t.token[path[0]] if path else final
        counts[first] += 1
    tv = 0.5 * np.abs(counts / n - p).sum()
    assert tv < 0.03, tv


def _brute_inverse_cdf(w, u):
    # first index whose exact prefix sum exceeds u * total (Fractions: no rounding anywhere)
    from fractions import Fraction
    fw = [Fraction(float(x)) for x in w]
    target = Fraction(float(u)) * sum(fw)
    run = Fraction(0)
    for i, x in enumerate(fw):
        run += x
        if run > target:
            return i
    return max(i for i, x in enumerate(fw) if x > 0)


@pytest.mark.parametrize('V', [1, 5, 300, 20000, 151936])
def test_draws_equal_brute_force_inverse_cdf(V):
    rng = np.random.default_rng(V)
    w = rng.exponential(size=V)
    w[rng.random(V) < 0.3] = 0.0             # zero weights inside chunks
    if not (w > 0).any():
        w[0] = 1.0
    checked = 0
    for u in list(rng.random(20 if V < 50000 else 6)) + [0.0, 1.0 - 2.0 ** -53]:
        exp = _brute_inverse_cdf(w, u)
        for fn in (ref.draw, ref.draw3):
            tok, margin = fn(w, u)
            if margin > 1e-12:
                assert tok == exp, (fn.__name__, u)
                checked += 1
    assert checked > 0


def test_draw3_fallbacks():
    assert ref.draw3(np.zeros(7), 0.3)[0] == 0                       # nothing positive: token 0
    w = np.zeros(40000); w[12345] = 2.0
    assert ref.draw3(w, 0.999999)[0] == 12345                        # single positive entry in a late chunk
    w = np.zeros(300); w[[3, 250]] = 1.0
    assert ref.draw3(w, 1.0 - 2.0 ** -53)[0] == 250                  # target at the very top: last positive


def test_walk_thresholds_follow_the_iterative_residual():
    # each trial's acceptance threshold in the walk is r_j(x) / q(x) with r_j renormalised max(r_{j-1} - q, 0):
    # a uniform just below it accepts, just above it rejects (pins the c_j closed form against the definition)
    rng = np.random.default_rng(5)
    V = 12
    for _ in range(6):
        pl = rng.normal(size=V).astype(np.float32) * 2
        ql = rng.normal(size=V).astype(np.float32) * 2
        T = 0.8
        p = ref.softmax_weights(pl, T); p /= p.sum()
        q = ref.softmax_weights(ql, T); q /= q.sum()
        xs = [int(x) for x in rng.choice(V, size=4, replace=True, p=q)]
        t = flatten(0, [[x] for x in xs])
        tree = dict(token=t.token, trial_start=t.trial_start, n_trials=t.n_trials, trials=t.trials)
        P, Q = np.stack([pl] * t.size), np.stack([ql] * t.size)
        r, ratios = p.copy(), []
        for x in xs:
            ratios.append(r[x] / q[x])
            d = np.maximum(r - q, 0.0)
            r = d / d.sum()
        for j, rho in enumerate(ratios):
            if rho >= 1.0 or rho < 1e-6:
                continue
            for factor, accept in ((1 - 1e-9, True), (1 + 1e-9, False)):
                u = [1.0 - 2.0 ** -53] * j + [rho * factor, 0.5, 0.5]
                path, final, used, bonus, _ = ref.accept_tree(P, Q, tree, u, T, 1)
                if accept:
                    assert path and t.token[path[0]] == xs[j] and used == j + 2 and bonus
                else:
                    assert used >= j + 2 and (not path or t.token[path[0]] != xs[j] or xs.count(xs[j]) > 1)
        # all rejected: the final draw follows the last residual
        u = [1.0 - 2.0 ** -53] * len(xs) + [0.37]
        if all(rho < 1.0 - 1e-9 for rho in ratios):
            path, final, used, bonus, margin = ref.accept_tree(P, Q, tree, u, T, 1)
            assert not path and not bonus and used == len(xs) + 1
            if margin > 1e-9:
                assert final == _brute_inverse_cdf(r, 0.37)


def test_first_argmax_is_pythons_max_rule():
    # speculative.py:68,80 pick max(range(n), key=logits.__getitem__): the first maximal index
    rng = random.Random(4)
    for _ in range(500):
        v = [rng.choice([0.0, 0.5, 1.0, -1.0]) for _ in range(rng.randint(1, 9))]
        assert ref.first_argmax(v) == max(range(len(v)), key=v.__getitem__)
