"""Engine-level parity of the HIP decode path against the CPU oracle (fp16-class tolerance, greedy identity where the
oracle's top-2 margin exceeds it), plus the invariants the reference fixes: position handling, window rule,
batch == independent sequences, graph replay == eager."""
import pytest
import torch

from oracle.qwen_ref import RefQwen2, max_rel, top2_margin
from seedplane_amd.presets import preset
from seedplane_amd.qwen_engine import Qwen2Engine
from seedplane_amd.synth import make_weights, random_prompt
from tests.conftest import small_cfg

pytestmark = pytest.mark.gpu

TOL = 2e-2     # max |a - b| / max |b| for fp16-class paths


def _fp16_rounded(w):
    """The GPU runs float checkpoints with fp16 matrices: give the oracle the same rounded matrices."""
    return {k: (v.half().float() if v.dim() == 2 else v.float()) for k, v in w.items()}


def _check_greedy(tokens, ref_rows, tol=TOL):
    """Greedy ids must equal the oracle's wherever the oracle's top-2 margin exceeds tol * max|logit|."""
    for i, (t, row) in enumerate(zip(tokens, ref_rows)):
        r = int(torch.argmax(row))
        if t != r:
            assert top2_margin(row) <= tol * float(row.abs().max()), f'step {i}: {t} vs {r}'


@pytest.fixture(scope='module')
def tiny(gpu_device):
    cfg, w = make_weights(preset('tiny'), 'f32', seed=0)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=16)
    ref = RefQwen2(cfg, _fp16_rounded(w))
    return cfg, eng, ref


@pytest.fixture(scope='module', params=['q8', 'q4', 'f16'])
def small(gpu_device, request):
    cfg, w = make_weights(small_cfg(), request.param, seed=11)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=64)
    ref = RefQwen2(cfg, w)
    return request.param, cfg, eng, ref


def test_tiny_prefill_and_decode_logits(tiny):
    cfg, eng, ref = tiny
    print('tiny prefill/decode', flush=True)
    ids = [1, 2, 3, 4, 5, 6, 7, 49, 0]
    lg, cache = eng.forward(ids, eng.new_cache(32), all_logits=True)
    rc = ref.new_cache(32)
    rl = ref.forward(ids, rc, all_logits=True)
    assert max_rel(lg, rl) < TOL
    for t in [3, 17, 42, 8]:
        lg, cache = eng.forward([t], cache)
        rl = ref.forward([t], rc)
        assert max_rel(lg[-1], rl[-1]) < TOL


def test_explicit_positions_match_default_and_shift_changes_logits(tiny):
    # the reference's tests/test_core.py:168-175 through the HIP engine
    cfg, e, _ = tiny
    ids = [1, 2, 3, 4]
    a, _ = e.forward(ids, e.new_cache(8), all_logits=True)
    b, _ = e.forward(ids, e.new_cache(8), all_logits=True, positions=[0, 1, 2, 3])
    c, _ = e.forward(ids, e.new_cache(8), all_logits=True, positions=[0, 40, 41, 42])
    assert torch.equal(a, b)
    assert float((a - c).abs().max()) > 1e-4


def test_errors_match_reference_classes(tiny):
    cfg, e, _ = tiny
    with pytest.raises(ValueError):
        e.forward([], e.new_cache(8))
    with pytest.raises(ValueError):
        e.forward([1, 2, 3], e.new_cache(2))
    with pytest.raises(ValueError):
        e.forward([1, 2], e.new_cache(8), positions=[0])
    with pytest.raises(ValueError):
        e.new_cache(0)


def test_small_models_match_oracle_greedy(small):
    fmt, cfg, eng, ref = small
    print(f'small {fmt} greedy', flush=True)
    prompt = random_prompt(20, cfg['vocab_size'], seed=5)
    toks = list(eng.generate(prompt, max_new_tokens=12))
    rows = ref.teacher_forced(prompt, toks)
    _check_greedy(toks, rows)
    lg, _ = eng.forward(prompt + toks[:-1], eng.new_cache(64), all_logits=True)
    rl = ref.forward(prompt + toks[:-1], ref.new_cache(64), all_logits=True)
    assert max_rel(lg, rl) < TOL, fmt


def test_windowed_ring_matches_windowed_oracle(small):
    fmt, cfg, eng, ref = small
    print(f'window {fmt}', flush=True)
    W = 8
    ids = random_prompt(30, cfg['vocab_size'], seed=9)
    cache = eng.new_cache(4096, window=W)
    # feed in uneven chunks so ring wrap happens inside multi-token calls and between calls
    out = []
    for a, b in [(0, 5), (5, 6), (6, 17), (17, 18), (18, 30)]:
        lg, cache = eng.forward(ids[a:b], cache, all_logits=True)
        out.append(lg)
    lg = torch.cat(out)
    rl = ref.forward(ids, ref.new_cache(30), all_logits=True, window=W)
    assert max_rel(lg, rl) < TOL
    full = ref.forward(ids, ref.new_cache(30), all_logits=True)
    assert max_rel(full[-1], rl[-1]) > 10 * max_rel(lg[-1], rl[-1])   # the window mattered


def test_batch_equals_independent_sequences(small):
    fmt, cfg, eng, _ = small
    prompts = [random_prompt(n, cfg['vocab_size'], seed=n) for n in (3, 17, 9)]
    batched = eng.generate_batch(prompts, max_new_tokens=6, graph=False)
    for p, b in zip(prompts, batched):
        single = list(eng.generate(p, max_new_tokens=6))
        assert single == b, fmt


def test_graph_replay_matches_eager(small):
    fmt, cfg, eng, _ = small
    prompts = [random_prompt(n, cfg['vocab_size'], seed=100 + n) for n in (4, 7)]
    eager = eng.generate_batch(prompts, max_new_tokens=8, graph=False)
    for _ in range(3):                    # replays with eager work in between
        graphed = eng.generate_batch(prompts, max_new_tokens=8, graph=True)
        assert graphed == eager
        assert eng.generate_batch(prompts, max_new_tokens=3, graph=False) == [e[:3] for e in eager]


def test_new_cache_growth_keeps_live_caches(small):
    # the reference's caches are independent tensors (qwen_engine.py:82-85): making more caches, with more slots,
    # must not disturb one that is in use
    fmt, cfg, eng, ref = small
    print(f'cache growth {fmt}', flush=True)
    ids = random_prompt(40, cfg['vocab_size'], seed=31)
    a = eng.new_cache(48)
    w = eng.new_cache(4096, window=8)
    eng.forward(ids[:20], a)
    eng.forward(ids[:20], w)
    n0, s0 = eng._pool_n, eng._pool_slots
    more = []
    while eng._pool_n == n0:                                  # more sequences than the pool holds: it grows...
        more.append(eng.new_cache(16))
    more.append(eng.new_cache(s0 + 200))                      # ... and then in slots (every ring slot moves)
    assert eng._pool_slots > s0
    assert a.epoch == eng._epoch and w.epoch == eng._epoch
    lg, _ = eng.forward(ids[20:], a, all_logits=True)
    lw, _ = eng.forward(ids[20:], w, all_logits=True)
    rl = ref.forward(ids, ref.new_cache(40), all_logits=True)[20:]
    rw = ref.forward(ids, ref.new_cache(40), all_logits=True, window=8)[20:]
    assert max_rel(lg, rl) < TOL
    assert max_rel(lw, rw) < TOL
    for c in more:                                            # the new caches work too
        out, _ = eng.forward(ids[:3], c)
        assert torch.isfinite(out).all()


def test_cache_tensors_read_back_in_reference_layout(small):
    """KVCache.keys[l] / values[l] (reference: per-layer [1, capacity, kv_heads, head_dim] tensors) read back the
    engine's ring: the oracle's cached (rotated) keys and values at every written position, zeros after `length`;
    a windowed cache holds its last n_slots positions.  Copies: writing one leaves the cache unchanged."""
    fmt, cfg, eng, ref = small
    ids = random_prompt(21, cfg['vocab_size'], seed=31)
    cache = eng.new_cache(40)
    eng.forward(ids[:13], cache)
    for t in ids[13:]:
        eng.decode([t], [cache])
    rc = ref.new_cache(40)
    ref.forward(ids, rc)
    L, NKV, HD = cfg['num_hidden_layers'], cfg['num_key_value_heads'], cfg['hidden_size'] // cfg['num_attention_heads']
    assert len(cache.keys) == len(cache.values) == L
    n = len(ids)
    for l in range(L):
        k, v = cache.keys[l], cache.values[l]
        assert k.shape == (1, 40, NKV, HD) and k.dtype == torch.float16
        assert max_rel(k[0, :n].float().cpu(), rc.keys[l][0, :n]) < TOL, l
        assert max_rel(v[0, :n].float().cpu(), rc.values[l][0, :n]) < TOL, l
        assert not k[0, n:].any() and not v[0, n:].any()
    k0 = cache.keys[-1].clone()
    cache.keys[-1].zero_()
    assert torch.equal(cache.keys[-1], k0)
    W = 8
    wc = eng.new_cache(4096, window=W)
    eng.forward(ids, wc)
    S = eng.slots_for(4096, W)
    first = max(0, n - S)
    for l in (0, L - 1):
        k = wc.keys[l]
        assert k.shape[1] == 4096
        assert not k[0, :first].any()
        # layer 0's keys depend only on each position's own token, so the ring holds the full cache's keys there
        if l == 0:
            assert max_rel(k[0, first:n].float().cpu(), rc.keys[0][0, first:n]) < TOL
