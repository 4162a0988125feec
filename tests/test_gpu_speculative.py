"""Speculative verification on the GPU against the oracle: seeded draws and tree acceptance bit-exact given identical
logits and uniforms (every compared decision is checked to lie outside rounding of its threshold), tree-masked
logits equal linear causal logits of each root path, greedy tree verification equals the reference verify_greedy,
and the KV compaction keeps later decoding consistent."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import speculative_ref as sref
from oracle.qwen_ref import RefQwen2, max_rel, top2_margin
from seedplane_amd import _lib
from seedplane_amd.qwen_engine import Qwen2Engine
from seedplane_amd.speculative import (SpecStats, SpeculativeForest, TreeDrafter, TreeVerifier, flatten, sample_rows,
                                       speculative_generate, uniforms)
from seedplane_amd.synth import make_weights, random_prompt
from tests.conftest import small_cfg

pytestmark = pytest.mark.gpu
TOL = 2e-2
MARGIN = 1e-12


@pytest.fixture(scope='module')
def model(gpu_device):
    cfg, w = make_weights(small_cfg(), 'q8', seed=21)
    return cfg, w, Qwen2Engine(config=cfg, tensors=w, max_tokens=64), RefQwen2(cfg, w)


@pytest.mark.parametrize('V,T', [(50, 0.8), (151936, 0.8), (151936, 1.0), (1000, 0.3)])
def test_sample_matches_oracle(gpu_device, V, T):
    print(f'sample V={V} T={T}', flush=True)
    g = torch.Generator().manual_seed(V)
    logits = torch.randn(4, V, generator=g) * 3
    rows = [0, 1, 2, 3, 0, 0, 1]
    u = sref.uniforms(5, V, len(rows))
    got = sample_rows(_lib.load(), logits.to(gpu_device), rows, u, T)
    for s, r in enumerate(rows):
        tok, margin = sref.draw(sref.softmax_weights(logits[r].numpy(), T), u[s])
        assert margin > MARGIN
        assert got[s] == tok, (s, r)


@pytest.mark.parametrize('V,n,T', [(300000, 600, 0.7), (2200000, 3, 1.0)])
def test_sample_windows_and_batches(gpu_device, V, n, T):
    """More draws than one launch sequence takes (512), chunks longer than a sum block's LDS window (V = 300000: 8
    chunks of 293 entries per block), a chunk longer than the draw's scan window (V = 2200000: 2149 entries)."""
    print(f'sample V={V} n={n} T={T}', flush=True)
    g = torch.Generator().manual_seed(V + n)
    logits = torch.randn(4, V, generator=g) * 2
    rows = [int(r) for r in torch.randint(0, 4, (n,), generator=g)]
    u = sref.uniforms(7, V, n)
    got = sample_rows(_lib.load(), logits.to(gpu_device), rows, u, T)
    w = [sref.softmax_weights(logits[r].numpy(), T) for r in range(4)]
    for s, r in enumerate(rows):
        tok, margin = sref.draw(w[r], u[s])
        assert margin > MARGIN
        assert got[s] == tok, (s, r)


def test_sample_zero_weight_chunks(gpu_device):
    """A row whose weights underflow to zero everywhere but one spike (every chunk before it sums to zero, every
    prefix after it is the total), and a row of equal logits (every entry drawable)."""
    V = 151936
    logits = torch.zeros(2, V)
    logits[0, 123457] = 50.0
    u = [0.0, 0.25, 0.999999, 0.5, 0.0, 0.3, 0.7, 0.999]
    rows = [0, 0, 0, 0, 1, 1, 1, 1]
    got = sample_rows(_lib.load(), logits.to(gpu_device), rows, u, 0.05)
    assert got[:4] == [123457] * 4
    w1 = sref.softmax_weights(logits[1].numpy(), 0.05)
    for s in range(4, 8):
        assert got[s] == sref.draw(w1, u[s])[0]
    assert got[4] == 0


def _random_case(rng, V, n_branches=8, depth=4, noise=0.3):
    branches = [[int(rng.integers(0, min(V, 6))) if rng.random() < 0.5 else int(rng.integers(0, V))
                 for _ in range(depth)] for _ in range(n_branches)]
    tree = flatten(int(rng.integers(0, V)), branches)
    base = rng.normal(size=(tree.size, V)).astype(np.float32) * 2
    for i in range(1, tree.size):          # make the target like the drafted tokens, so some trials accept
        base[tree.parent[i], tree.token[i]] += 3.0
    p = base
    q = (base + rng.normal(size=base.shape).astype(np.float32) * noise).astype(np.float32)
    return tree, p, q


@pytest.mark.parametrize('V', [64, 151936])
def test_accept_tree_matches_oracle(model, V):
    cfg, w, eng, _ = model
    verifier = TreeVerifier(eng)
    rng = np.random.default_rng(V)
    accepted_total = 0
    for case in range(12 if V < 1000 else 4):
        print(f'accept V={V} case={case}', flush=True)
        tree, p, q = _random_case(rng, V)
        u = sref.uniforms(9, case, 64)
        dev = eng.device
        got = verifier.accept(torch.from_numpy(p).to(dev), torch.from_numpy(q).to(dev), tree, u, 0.8)
        t = dict(token=tree.token, trial_start=tree.trial_start, n_trials=tree.n_trials, trials=tree.trials)
        path, final, used, bonus, margin = sref.accept_tree(p, q, t, u, 0.8, tree.max_depth)
        assert margin > MARGIN
        assert (got[0], got[1], got[2], got[3]) == (path, final, used, bonus)
        accepted_total += len(path)
    assert accepted_total > 0       # the cases exercise acceptance, not only rejection



def _accept_device_entry(eng, pd, qd, tree, u, T):
    """sp_op_accept_tree with the tree arrays and uniforms in device memory."""
    dev = eng.device
    md = max(1, tree.max_depth)
    arrs = [torch.tensor(np.asarray(x, dtype=np.int32), device=dev)
            for x in (tree.token, tree.trial_start, tree.n_trials, tree.trials if len(tree.trials) else [0])]
    ud = torch.tensor(np.asarray(u, dtype=np.float64), device=dev)
    out = torch.empty(md + 4, dtype=torch.int32, device=dev)
    res = np.empty(md + 4, dtype=np.int32)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    _lib.check(eng.lib.sp_op_accept_tree(ptr(pd), ptr(qd), pd.shape[1], pd.stride(0), tree.size, *[ptr(a) for a in arrs],
                                         len(tree.trials), ptr(ud), len(u), float(T), md, None, ptr(out), stream,
                                         res.ctypes.data_as(ctypes.c_void_p)))
    torch.cuda.synchronize()
    o = res.tolist()
    assert o == out.cpu().tolist()
    return o[1:1 + o[0]], o[md + 1], o[md + 2], bool(o[md + 3])


@pytest.mark.parametrize('V', [64, 151936])
def test_accept_tree_entries_agree(model, V):
    """The device-array and host-array entry points take the same decisions (and the oracle's), including (small
    vocabulary) a walk that consumes more uniforms than the kernel stages in LDS: 300 rejected trials of one child.
    (With q = p off that child every other token has the same ratio p / q, so once c_j reaches it the residual is
    rounding noise of p - c_j q; at 151936 entries that noise, not the rule, would pick the final token.)"""
    cfg, w, eng, _ = model
    verifier = TreeVerifier(eng)
    rng = np.random.default_rng(V + 1)
    dev = eng.device
    cases = [_random_case(rng, V) for _ in range(3)]
    if V < 1000:
        # one child drawn 300 times, far more likely under q than under p: every trial is rejected
        tree = flatten(1, [[2]] * 300)
        p = rng.normal(size=(tree.size, V)).astype(np.float32)
        q = p.copy()
        p[0, 2] -= 8.0
        q[0, 2] += 8.0
        cases.append((tree, p, q))
    for case, (tree, p, q) in enumerate(cases):
        print(f'entries V={V} case={case}', flush=True)
        u = sref.uniforms(11, case, 400)
        pd, qd = torch.from_numpy(p).to(dev), torch.from_numpy(q).to(dev)
        got_dev = _accept_device_entry(eng, pd, qd, tree, u, 0.8)
        got_host = verifier.accept(pd, qd, tree, u, 0.8)
        t = dict(token=tree.token, trial_start=tree.trial_start, n_trials=tree.n_trials, trials=tree.trials)
        path, final, used, bonus, margin = sref.accept_tree(p, q, t, u, 0.8, tree.max_depth)
        assert margin > MARGIN
        assert tuple(got_dev) == tuple(got_host) == (path, final, used, bonus)
        if case == 3:
            assert path == [] and used == 301

def test_accept_tree_rows_by_index(model):
    """sp_op_accept_tree_rows with the drafter rows scattered over a larger buffer takes the decisions of the
    host-array entry over the same rows gathered in node order, and refuses an index past the buffer."""
    cfg, w, eng, _ = model
    verifier = TreeVerifier(eng)
    rng = np.random.default_rng(5)
    dev = eng.device
    for case in range(4):
        tree, p, q = _random_case(rng, 151936 if case == 0 else 64)
        V = p.shape[1]
        nr = tree.size + 7
        perm = rng.permutation(nr)[:tree.size]               # node i's row in the scattered buffer
        big = rng.normal(size=(nr, V)).astype(np.float32)
        big[perm] = q
        u = sref.uniforms(13, case, 64)
        pd = torch.from_numpy(p).to(dev)
        got_rows = verifier.accept(pd, torch.from_numpy(big).to(dev), tree, u, 0.8, q_index=perm.tolist())
        got_host = verifier.accept(pd, torch.from_numpy(q).to(dev), tree, u, 0.8)
        assert tuple(got_rows) == tuple(got_host), case
    bad = perm.copy()
    bad[0] = nr                                               # the root has trials: its row is read
    with pytest.raises(ValueError, match='malformed tree'):
        verifier.accept(pd, torch.from_numpy(big).to(dev), tree, u, 0.8, q_index=bad.tolist())


def _link_ref(toks, nb, level, canon):
    """Host restatement of one sp_op_draft_link level (first branch with the same prefix; canonical ancestors)."""
    c = []
    for b in range(nb):
        cb = next(o for o in range(b + 1) if all(toks[lv][o] == toks[lv][b] for lv in range(level + 1)))
        c.append(cb)
    canon[level] = c
    masks = [(1 << (level * nb + b)) | sum(1 << (lv * nb + canon[lv][b]) for lv in range(level)) for b in range(nb)]
    return c, masks


def test_draft_link_matches_host_rule(gpu_device):
    lib = _lib.load()
    rng = np.random.default_rng(3)
    for nb, depth in [(8, 4), (5, 3), (1, 5), (16, 4)]:
        toks = rng.integers(0, 3, size=(depth, nb)).astype(np.int32)     # few values: many shared prefixes
        td = torch.from_numpy(toks).to(gpu_device)
        canon = torch.full((depth, nb), -1, dtype=torch.int32, device=gpu_device)
        masks = torch.zeros(nb, dtype=torch.int64, device=gpu_device)
        rows = torch.zeros(nb, dtype=torch.int32, device=gpu_device)
        ref_canon = [[0] * nb for _ in range(depth)]
        ptr = lambda t: ctypes.c_void_p(t.data_ptr())
        for level in range(depth - 1):
            _lib.check(lib.sp_op_draft_link(ptr(td), nb, level, ptr(canon), ptr(masks), ptr(rows), None))
            c, m = _link_ref(toks.tolist(), nb, level, ref_canon)
            assert canon[level].tolist() == c and rows.tolist() == c
            assert [int(x) & (2 ** 64 - 1) for x in masks.tolist()] == m, (nb, level)
    assert lib.sp_op_draft_link(ptr(td), 16, 4, ptr(canon), ptr(masks), ptr(rows), None) == _lib.SP_EINVAL


def test_device_drafter_rows_and_draws(model, gpu_device):
    """The device-side proposal: every drafted prefix's row equals the drafter run linearly over that prefix
    (fp16 bar), branches sharing a prefix share its row, and each branch's token at every level is the oracle's draw
    from its prefix's row with the level's uniform (bit-exact)."""
    cfg, w, eng, _ = model
    drafter = TreeDrafter(eng)
    prefix = random_prompt(11, cfg['vocab_size'], seed=12)
    B, depth, T = 8, 4, 1.5
    u = sref.uniforms(21, 0, B * depth + 8)
    cache = eng.new_cache(128)
    eng.forward(prefix[:-1], cache)
    branches, rows, used = drafter.propose(cache, [prefix[-1]], B, depth, T, u)
    assert used == B * depth and len(branches) == B and all(len(b) == depth for b in branches)
    assert cache.length == len(prefix)
    for b in range(B):
        for lv in range(depth):
            pref = tuple(branches[b][:lv])
            row = rows[pref].cpu()
            tok, margin = sref.draw(sref.softmax_weights(row.numpy(), T), u[lv * B + b])
            assert margin > MARGIN and branches[b][lv] == tok, (b, lv)
    for pref, row in rows.items():
        lin, _ = eng.forward(prefix + list(pref), eng.new_cache(64), all_logits=True)
        assert max_rel(row, lin[-1]) < TOL, pref
    tree = flatten(prefix[-1], branches)
    idx = drafter.q_index(tree)
    prefixes = [()]
    for i in range(1, tree.size):
        prefixes.append(prefixes[tree.parent[i]] + (tree.token[i],))
    for i, pref in enumerate(prefixes):
        if tree.n_children[i]:
            assert torch.equal(drafter.q_rows[idx[i]], rows[pref])


def test_devcols_flag_errors(model):
    cfg, w, eng, _ = model
    cache = eng.new_cache(16)
    col = eng._column(1, cache, 0, 0)
    _lib.check(eng.lib.sp_engine_set_device_columns(eng.h, None, None), eng.h)
    with pytest.raises(RuntimeError, match='sp_engine_set_device_columns'):
        eng.run([col], _lib.SP_F_LOGITS | _lib.SP_F_DEVCOLS)
    t = torch.zeros(1, dtype=torch.int32, device=eng.device)
    _lib.check(eng.lib.sp_engine_set_device_columns(eng.h, ctypes.c_void_p(t.data_ptr()), None), eng.h)
    with pytest.raises(ValueError, match='both name the tokens'):
        eng.run([col], _lib.SP_F_LOGITS | _lib.SP_F_DEVCOLS | _lib.SP_F_FEED)
    _lib.check(eng.lib.sp_engine_set_device_columns(eng.h, None, None), eng.h)


def test_tree_pass_equals_linear_paths(model):
    cfg, w, eng, _ = model
    prefix = random_prompt(12, cfg['vocab_size'], seed=4)
    branches = [[3, 4, 5], [3, 4, 9], [3, 7], [11, 12, 13, 14]]
    verifier = TreeVerifier(eng)
    cache = eng.new_cache(64)
    eng.forward(prefix[:-1], cache)
    tree = flatten(prefix[-1], branches)
    out = torch.empty((tree.size, cfg['vocab_size']), dtype=torch.float32, device=eng.device)
    ids = verifier.forward(cache, tree, logits_out=out)
    assert cache.length == len(prefix) - 1
    for i in range(tree.size):
        path, j = [], i
        while j > 0:
            path.append(tree.token[j]); j = tree.parent[j]
        seq = prefix + path[::-1]
        lin, _ = eng.forward(seq, eng.new_cache(64), all_logits=True)
        assert max_rel(out[i], lin[-1]) < TOL, i
        if int(ids[i]) != int(torch.argmax(lin[-1])):
            assert top2_margin(lin[-1]) <= TOL * float(lin[-1].abs().max())


def test_greedy_tree_verification_equals_reference_semantics(model):
    cfg, w, eng, ref = model
    prefix = random_prompt(10, cfg['vocab_size'], seed=8)
    greedy, _ = ref.generate_greedy(prefix, 4)
    branches = [greedy[:2] + [1, 2], greedy[:4], [greedy[0], 77], [5, 6], greedy[:3]]
    forest = SpeculativeForest.build(branches)

    def target_logits(seq):                      # reference contract: one position per call, from scratch
        c = ref.new_cache(len(seq))
        return ref.forward(list(seq), c)[-1].tolist()
    exp = sref.verify_greedy(prefix, sref.Forest.build(branches), target_logits)
    cache = eng.new_cache(64)
    eng.forward(prefix[:-1], cache)
    got = TreeVerifier(eng).verify_greedy(cache, prefix, forest)
    assert (got.emitted, got.accepted_draft_tokens, got.rejected, got.target_steps, got.branch) == exp
    # the cache now holds everything emitted except the last token: continue greedily and compare with a fresh run
    seq = prefix + list(got.emitted)
    assert cache.length == len(seq) - 1
    cont = []
    tok = seq[-1]
    for _ in range(4):
        tok = int(eng.decode([tok], [cache], graph=False)[0])
        cont.append(tok)
    fresh = list(eng.generate(seq, max_new_tokens=4))
    rows = ref.teacher_forced(seq, cont)
    for a, b, row in zip(cont, fresh, rows):
        if a != b:
            assert top2_margin(row) <= TOL * float(row.abs().max())


def test_identical_drafter_accepts_every_draft(model, gpu_device):
    cfg, w, eng, _ = model
    drafter = TreeDrafter(Qwen2Engine(config=cfg, tensors=w, max_tokens=64))
    stats = SpecStats()
    prompt = random_prompt(9, cfg['vocab_size'], seed=2)
    out = speculative_generate(eng, drafter, prompt, steps=4, n_branches=4, depth=3, temperature=0.8, seed=1,
                               stats=stats)
    # p == q up to fp16-class noise: every first trial accepts (u < ratio ~ 1) except near-ties, so nearly every
    # step keeps all `depth` drafts plus a bonus
    assert stats.steps == 4 and len(out) == stats.emitted
    assert stats.accepted >= 3 * stats.steps - 2


def test_linear_verify_with_rollback_matches_fresh_run(model):
    # benchmark_speculative.py:85-131: one batched pass over the draft, accept by row argmax, roll the cache back
    # by assigning length, continue with the correction; the cache must then equal a fresh run of the emitted tokens
    cfg, w, eng, ref = model
    prefix = random_prompt(11, cfg['vocab_size'], seed=12)
    greedy, _ = ref.generate_greedy(prefix, 5)
    for draft in (greedy[:4], greedy[:2] + [7, 8], [9] + greedy[1:4]):
        cache = eng.new_cache(64)
        pre, _ = eng.forward(prefix, cache)
        pre_id = int(torch.argmax(pre[-1]))
        old = cache.length
        block, _ = eng.forward(draft, cache, all_logits=True)
        block_ids = [int(torch.argmax(r)) for r in block]
        emitted, accepted, keep = sref.linear_verify(draft, pre_id, block_ids)
        cache.length = old + keep
        if len(emitted) > keep:                       # a correction token follows the kept drafts
            nxt, _ = eng.forward([emitted[-1]], cache)
        else:
            nxt = block[-1:]
        fresh, _ = eng.forward(prefix + emitted, eng.new_cache(64))
        assert cache.length == len(prefix) + len(emitted)
        assert max_rel(nxt[-1], fresh[-1]) < TOL, draft
        exp_emitted = []                              # greedy reference semantics of the same rule
        for i, d in enumerate(draft):
            exp_emitted.append(greedy[i])
            if d != greedy[i]:
                break
        if all(top2_margin(r) > TOL * float(r.abs().max()) for r in ref.teacher_forced(prefix, greedy[:5])):
            assert emitted == exp_emitted, (draft, emitted, exp_emitted)


def test_logits_only_pass_returns_the_engine_rows_without_a_copy(model):
    # ids=False without logits_out hands back a view of the engine's own logits buffer; it equals the copied rows
    cfg, w, eng, _ = model
    prefix = random_prompt(9, cfg['vocab_size'], seed=14)
    tree = flatten(prefix[-1], [[1, 2, 3], [1, 5], [7]])
    verifier = TreeVerifier(eng)
    cache = eng.new_cache(64)
    eng.forward(prefix[:-1], cache)
    copied = torch.empty((tree.size, cfg['vocab_size']), dtype=torch.float32, device=eng.device)
    verifier.forward(cache, tree, logits_out=copied)
    view = verifier.forward(cache, tree, ids=False)
    assert view.shape == copied.shape and view.dtype == torch.float32
    ptr = ctypes.c_void_p()
    _lib.check(eng.lib.sp_engine_logits(eng.h, ctypes.byref(ptr)), eng.h)
    assert view.data_ptr() == ptr.value
    assert torch.equal(view, copied)


def test_library_release_then_reuse(model, gpu_device):
    """sp_library_release frees the sampling and acceptance scratch; the next calls create it again and give the
    same draws and decisions."""
    cfg, w, eng, _ = model
    lib = _lib.load()
    g = torch.Generator().manual_seed(1)
    logits = (torch.randn(3, 5000, generator=g) * 2).to(gpu_device)
    u = sref.uniforms(2, 0, 6)
    first = sample_rows(lib, logits, [0, 1, 2, 0, 1, 2], u, 0.9)
    tree, p, q = _random_case(np.random.default_rng(8), 64)
    pd, qd = torch.from_numpy(p).to(gpu_device), torch.from_numpy(q).to(gpu_device)
    verifier = TreeVerifier(eng)
    ua = sref.uniforms(4, 0, 64)
    a1 = verifier.accept(pd, qd, tree, ua, 0.8)
    assert lib.sp_library_release() == _lib.SP_OK
    assert lib.sp_library_release() == _lib.SP_OK          # nothing held: no-op
    assert sample_rows(lib, logits, [0, 1, 2, 0, 1, 2], u, 0.9) == first
    assert verifier.accept(pd, qd, tree, ua, 0.8) == a1
