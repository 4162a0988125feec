"""Pins of the CPU oracle (oracle/qwen_ref.py, oracle/quant_ref.py) that do not need a GPU."""
import math

import pytest
import torch

from oracle.qwen_ref import RefQwen2, tree_attention_mask
from oracle.quant_ref import dequant_q4, dequant_q8, unpack_q4
from seedplane_amd.presets import preset
from seedplane_amd.synth import make_weights
from tests.conftest import small_cfg


def _hf_model(cfg, w, sliding_window=None):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    kw = {}
    if sliding_window is not None:
        kw = dict(use_sliding_window=True, sliding_window=sliding_window, max_window_layers=0)
    hc = Qwen2Config(vocab_size=cfg['vocab_size'], hidden_size=cfg['hidden_size'],
                     intermediate_size=cfg['intermediate_size'], num_hidden_layers=cfg['num_hidden_layers'],
                     num_attention_heads=cfg['num_attention_heads'], num_key_value_heads=cfg['num_key_value_heads'],
                     max_position_embeddings=cfg['max_position_embeddings'], rope_theta=cfg['rope_theta'],
                     rms_norm_eps=cfg['rms_norm_eps'], tie_word_embeddings=True, attn_implementation='eager', **kw)
    m = Qwen2ForCausalLM(hc).eval()
    m.load_state_dict({k: v.float() for k, v in w.items()}, strict=False)
    m.tie_weights()
    return m


def test_oracle_matches_transformers_on_tiny_fixture(tiny_f32):
    # The reference validated Qwen2Engine against Transformers (experiments/v17/validate.py:10-29, 2.29e-5).
    cfg, w = tiny_f32
    ref = RefQwen2(cfg, w)
    m = _hf_model(cfg, w)
    ids = [1, 2, 3, 4, 5, 6, 7, 49, 0]
    with torch.no_grad():
        hf = m(torch.tensor([ids])).logits[0]
    ours = ref.forward(ids, ref.new_cache(16), all_logits=True)
    assert float((hf - ours).abs().max() / hf.abs().max()) < 1e-5


def test_oracle_decode_matches_prefill(tiny_f32):
    # token-by-token decode through the cache equals the one-shot causal pass
    cfg, w = tiny_f32
    ref = RefQwen2(cfg, w)
    ids = [3, 9, 27, 1, 4]
    full = ref.forward(ids, ref.new_cache(8), all_logits=True)
    c = ref.new_cache(8)
    rows = [ref.forward([t], c)[-1] for t in ids]
    assert float((torch.stack(rows) - full).abs().max()) < 1e-4


def test_explicit_positions_match_default_and_shift_changes_logits(tiny_f32):
    # restatement of the reference's tests/test_core.py:168-175 on the oracle
    cfg, w = tiny_f32
    e = RefQwen2(cfg, w)
    ids = [1, 2, 3, 4]
    a = e.forward(ids, e.new_cache(8), all_logits=True)
    b = e.forward(ids, e.new_cache(8), all_logits=True, positions=[0, 1, 2, 3])
    c = e.forward(ids, e.new_cache(8), all_logits=True, positions=[0, 40, 41, 42])
    assert torch.equal(a, b)
    assert float((a - c).abs().max()) > 1e-4


def test_window_at_least_context_equals_full_attention(tiny_f32):
    cfg, w = tiny_f32
    e = RefQwen2(cfg, w)
    ids = list(range(1, 13))
    full = e.forward(ids, e.new_cache(12), all_logits=True)
    win = e.forward(ids, e.new_cache(12), all_logits=True, window=12)
    assert torch.equal(full, win)
    narrow = e.forward(ids, e.new_cache(12), all_logits=True, window=4)
    assert torch.equal(narrow[:4], full[:4])          # the first W positions see the same keys
    assert float((narrow[-1] - full[-1]).abs().max()) > 1e-4


def test_window_matches_transformers_sliding_window(tiny_f32):
    # Hugging Face rule kv_idx > q_idx - sliding_window pins the window semantics
    cfg, w = tiny_f32
    e = RefQwen2(cfg, w)
    ids = [5, 17, 2, 33, 8, 1, 40, 22, 19, 7, 3, 11]
    m = _hf_model(cfg, w, sliding_window=5)
    with torch.no_grad():
        hf = m(torch.tensor([ids])).logits[0]
    ours = e.forward(ids, e.new_cache(len(ids)), all_logits=True, window=5)
    full = e.forward(ids, e.new_cache(len(ids)), all_logits=True)
    assert float((hf - ours).abs().max() / hf.abs().max()) < 1e-5
    assert float((hf - full).abs().max()) > 1e-3        # the window really changed the result


def test_rmsnorm_closed_form(tiny_f32):
    cfg, w = tiny_f32
    e = RefQwen2(cfg, w)
    H = cfg['hidden_size']
    c = -3.5
    x = torch.full((1, 1, H), c)
    wt = torch.linspace(0.5, 2.0, H)
    out = e._norm(x, wt)[0, 0]
    expect = math.copysign(1.0, c) * abs(c) / math.sqrt(c * c + e.eps) * wt
    assert torch.allclose(out, expect, rtol=1e-6, atol=0)


def test_rope_identity_norm_and_relative_position(tiny_f32):
    cfg, w = tiny_f32
    e = RefQwen2(cfg, w)
    HD = e.head_dim
    g = torch.Generator().manual_seed(1)
    q = torch.randn(1, 1, 1, HD, generator=g)
    k = torch.randn(1, 1, 1, HD, generator=g)
    q0, k0 = e._rope(q, k, torch.tensor([0]))
    assert torch.equal(q0, q) and torch.equal(k0, k)
    qa, _ = e._rope(q, k, torch.tensor([37]))
    half = HD // 2
    pair = lambda t: t[..., :half] ** 2 + t[..., half:] ** 2      # non-interleaved pairs (i, i + HD/2)
    assert torch.allclose(pair(qa), pair(q), rtol=1e-5)
    # <R(p) q, R(p') k> depends on p - p' only
    def dot(p, pp):
        qr, _ = e._rope(q, k, torch.tensor([p]))
        _, kr = e._rope(q, k, torch.tensor([pp]))
        return float((qr * kr).sum())
    assert abs(dot(10, 3) - dot(107, 100)) < 1e-4
    assert abs(dot(10, 3) - dot(3, 10)) > 1e-3            # and not on |p - p'| only (sign of the rotation)


def test_dequant_closed_forms():
    codes = torch.tensor([[-127, -1, 0, 1, 127] + [5] * 27], dtype=torch.int8)
    scales = torch.tensor([[0.001953125]], dtype=torch.float16)   # 2^-9, exact
    wq = dequant_q8(codes, scales)
    assert wq[0, :5].tolist() == [-127 * 2 ** -9, -2 ** -9, 0.0, 2 ** -9, 127 * 2 ** -9]
    packed = torch.tensor([[0x21, 0xF0] + [0] * 14], dtype=torch.uint8)
    assert unpack_q4(packed)[0, :4].tolist() == [1, 2, 0, 15]       # even k in the low nibble
    sc = torch.tensor([[0.5]], dtype=torch.float16)
    z = torch.tensor([[7.5]], dtype=torch.float16)
    w4 = dequant_q4(packed, sc, z)
    assert w4[0, :4].tolist() == [(1 - 7.5) * 0.5, (2 - 7.5) * 0.5, -3.75, 3.75]


def test_tree_mask_logits_equal_linear_paths():
    # the target_logits contract (seedplane/speculative.py:58-61): a node's logits under the ancestor mask equal the
    # linear causal forward of its root path at positions prefix + depth
    cfg, w = make_weights(small_cfg(), 'q8', seed=3)
    e = RefQwen2(cfg, w)
    prefix = [11, 22, 33, 44, 55]
    toks = [7, 8, 9, 10, 12, 13]
    parents = [-1, 0, 0, 1, -1, 4]
    depth = [0, 1, 1, 2, 0, 1]
    c = e.new_cache(len(prefix) + len(toks))
    e.forward(prefix, c)
    allowed = tree_attention_mask(len(prefix), parents, depth=depth)
    tree = e.forward_masked(toks, c, [len(prefix) + d for d in depth], allowed)
    for i in range(len(toks)):
        path, j = [], i
        while j >= 0:
            path.append(toks[j]); j = parents[j]
        path = path[::-1]
        lc = e.new_cache(len(prefix) + len(path))
        lin = e.forward(prefix + path, lc, all_logits=True)[-1]
        assert float((lin - tree[i]).abs().max() / lin.abs().max()) < 1e-5, i


def test_synthetic_recipes_have_the_stated_statistics():
    cfg = small_cfg()
    _, w8 = make_weights(cfg, 'q8', seed=0)
    c = w8['model.layers.0.mlp.up_proj.qweight']
    assert c.dtype == torch.int8 and int(c.min()) >= -127 and int(c.max()) <= 127
    s = w8['model.layers.0.mlp.up_proj.scales'].float()
    assert float(s.min()) >= 0 and abs(float(s.pow(2).mean().sqrt()) - 0.002) < 2e-4
    _, w4 = make_weights(cfg, 'q4', seed=0)
    codes = unpack_q4(w4['model.layers.0.mlp.up_proj.qweight'])
    assert int(codes.min()) == 0 and int(codes.max()) == 15
    z = w4['model.layers.0.mlp.up_proj.qzeros'].float()
    assert float(z.min()) >= 7.0 and float(z.max()) <= 8.0
    # determinism
    _, again = make_weights(cfg, 'q8', seed=0)
    assert torch.equal(again['model.layers.1.self_attn.q_proj.qweight'], w8['model.layers.1.self_attn.q_proj.qweight'])


def test_storage_modes_round_where_they_say(tiny_f32):
    # 'fp16' is the reference at dtype float16 (qwen_engine.py:39-41), 'hip' rounds where the HIP engine stores fp16;
    # both stay within fp16 distance of the fp32 oracle, differ from it, and keep only fp16 values in the K/V cache
    cfg, w = tiny_f32
    ids = [1, 2, 3, 4, 5, 6, 7, 49, 0]
    base = RefQwen2(cfg, w).forward(ids, RefQwen2(cfg, w).new_cache(16), all_logits=True)
    for mode in ('fp16', 'hip'):
        ref = RefQwen2(cfg, w, storage=mode)
        c = ref.new_cache(16)
        lg = ref.forward(ids, c, all_logits=True)
        rel = float((lg - base).abs().max() / base.abs().max())
        assert 0 < rel < 2e-2, (mode, rel)
        for t in c.keys + c.values:
            assert torch.equal(t, t.half().float()), mode
    with pytest.raises(ValueError):
        RefQwen2(cfg, w, storage='bf16')
    with pytest.raises(ValueError):
        RefQwen2(cfg, w, storage={'kv', 'logits'})


def test_storage_points_compose(tiny_f32):
    # a set of storage points rounds exactly there: {'kv'} keeps fp16 values in the cache and differs from fp32;
    # 'x' is the union of its three consumers ('xq', 'xg', 'xh'); 'hip' is the union of every point
    cfg, w = tiny_f32
    ids = [1, 2, 3, 4, 5, 6, 7, 49, 0]

    def run(storage):
        ref = RefQwen2(cfg, w, storage=storage)
        c = ref.new_cache(16)
        return ref.forward(ids, c, all_logits=True), c

    base, c0 = run(None)
    kv, c1 = run({'kv'})
    assert not torch.equal(kv, base)
    for t in c1.keys + c1.values:
        assert torch.equal(t, t.half().float())
    assert any(not torch.equal(t, t.half().float()) for t in c0.keys)
    assert torch.equal(run({'x'})[0], run({'xq', 'xg', 'xh'})[0])
    assert not torch.equal(run({'xq'})[0], run({'x'})[0])
    assert torch.equal(run('hip')[0], run({'x', 'kv', 'attn', 'act'})[0])


def test_fp16_storage_matches_transformers_in_fp16(tiny_f32):
    # an independent fp16 execution of the same model: Transformers' Qwen2 with every tensor in float16
    cfg, w = tiny_f32
    ref = RefQwen2(cfg, w, storage='fp16')
    m = _hf_model(cfg, w).half()
    ids = [1, 2, 3, 4, 5, 6, 7, 49, 0]
    with torch.no_grad():
        hf = m(torch.tensor([ids])).logits[0].float()
    ours = ref.forward(ids, ref.new_cache(16), all_logits=True)
    assert float((hf - ours).abs().max() / hf.abs().max()) < 1e-2
