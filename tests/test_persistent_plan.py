"""The persistent one-column step's work split and bounds walk (host only, no GPU): sp_persistent_geometry builds the
geometry the engine launches with and runs the same walk the engine runs before its first launch -- every item's
block, every tagged word it reads or writes, every weight tile and staged count (d1::check_geom).  Checked here for
the shapes the GPU tests and the bench run, against independent counts of the work items, and for shapes it must
refuse."""
import ctypes

import pytest
import torch

from seedplane_amd import _lib
from seedplane_amd.presets import preset
from tests.conftest import small_cfg


def _desc(cfg, fmt):
    inv = (1.0 / (cfg['rope_theta'] ** (torch.arange(0, cfg['hidden_size'] // cfg['num_attention_heads'], 2).float()
                                         / (cfg['hidden_size'] // cfg['num_attention_heads'])))).numpy()
    buf = (ctypes.c_float * len(inv))(*inv)
    d = _lib.ModelDesc(cfg['num_hidden_layers'], cfg['hidden_size'], cfg['num_attention_heads'],
                       cfg['num_key_value_heads'], cfg['hidden_size'] // cfg['num_attention_heads'],
                       cfg['intermediate_size'], cfg['vocab_size'], fmt, 1, 64, 1e-6, 0.0,
                       ctypes.cast(buf, ctypes.POINTER(ctypes.c_float)))
    d._keep = buf
    return d


def _geometry(cfg, fmt, n_slots, n_blocks=256):
    lib = _lib.load()
    info = (ctypes.c_int32 * 12)()
    rc = lib.sp_persistent_geometry(ctypes.byref(_desc(cfg, fmt)), n_slots, n_blocks, info)
    return rc, list(info), lib.sp_last_error().decode()


@pytest.mark.parametrize('name,fmt,n_slots', [
    ('qwen2-1.5b', _lib.SP_FMT_Q8, 1024 + 64),      # the 1024 window of the int8 decode workload
    ('qwen2-1.5b', _lib.SP_FMT_Q8, 2048 + 64),      # decode at the 2048-token verify prefix
    ('qwen2-1.5b', _lib.SP_FMT_Q4, 1024 + 64),
    ('qwen2-0.5b', _lib.SP_FMT_F16, 576),           # the 16-request burst's pool
    ('qwen2-0.5b', _lib.SP_FMT_Q8, 576),
])
def test_model_shapes_fit_and_walk_clean(name, fmt, n_slots):
    cfg = preset(name)
    rc, info, err = _geometry(cfg, fmt, n_slots)
    assert rc == _lib.SP_OK, err
    nq, chunks, comb, no, nu, nd, nu_max, b2, b3, b5, words, lds = info
    H, I, NH, NKV = cfg['hidden_size'], cfg['intermediate_size'], cfg['num_attention_heads'], cfg['num_key_value_heads']
    HD = H // NH
    assert nq == (NH + 2 * NKV) * HD // 16 and no == H // 16 and nu == I // 16 and nd == 2 * (H // 16)
    assert chunks == NKV * -(-n_slots // 64) and comb == NH
    assert b2 == nq and b3 == 256 - no and b5 == 256 - nd
    assert b2 + chunks + comb <= 256                      # qkv tiles, chunks and combiners on distinct blocks
    assert nu_max == min(3, -(-nu // b3)) and nu <= 3 * b3 + no   # <= 3 units per block, overflow on o_proj blocks
    assert words == (NH + 2 * NKV) * HD + NH * (chunks // NKV) * (2 + HD) + NH * HD + H + I // 2 + 2 * H
    assert 80 * 1024 < lds <= 160 * 1024                  # one block per CU


def test_small_test_shapes_fit():
    for fmt in (_lib.SP_FMT_F16, _lib.SP_FMT_Q8, _lib.SP_FMT_Q4):
        rc, info, err = _geometry(small_cfg(), fmt, 16 + 4)
        assert rc == _lib.SP_OK, (fmt, err)
        rc, info, err = _geometry(preset('tiny'), fmt, 64)
        assert rc == _lib.SP_OK, (fmt, err)


def test_refused_shapes():
    # hidden 3584 (7B) exceeds the step's norm row; a pool whose chunks overflow the blocks; too few blocks
    assert _geometry(preset('qwen2-7b'), _lib.SP_FMT_Q4, 1088)[0] == _lib.SP_EINVAL
    rc, _, err = _geometry(preset('qwen2-1.5b'), _lib.SP_FMT_Q8, 4096)      # 64 chunks per kv head: 128 + 128 + 12 > 256
    assert rc == _lib.SP_EINVAL and 'blocks' in err
    rc, _, err = _geometry(preset('qwen2-1.5b'), _lib.SP_FMT_Q8, 8192)      # 128 chunks: more than one lane each
    assert rc == _lib.SP_EINVAL and 'chunks' in err
    assert _geometry(preset('qwen2-1.5b'), _lib.SP_FMT_Q8, 1088, n_blocks=120)[0] == _lib.SP_EINVAL
    # an fp16 1.5B shape needs 6 k-tiles per wave: no instantiation, so it runs the chain
    rc, _, err = _geometry(preset('qwen2-1.5b'), _lib.SP_FMT_F16, 1088)
    assert rc == _lib.SP_EINVAL and 'instantiation' in err
