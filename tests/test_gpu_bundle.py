"""A seedplane-bundle/2 directory loads into the HIP engine with the same results as the tensors it was written from
(bit-identical logits), and a float checkpoint quantized by the converter decodes within tolerance of the oracle run
on the bundle's own dequantised weights."""
import pytest
import torch

from oracle.quant_ref import dequant_all
from oracle.qwen_ref import RefQwen2, max_rel
from seedplane_amd import native_bundle
from seedplane_amd.qwen_engine import Qwen2Engine
from seedplane_amd.synth import make_weights, random_prompt, write_bundle
from tests.conftest import small_cfg
from tests.test_native_bundle import tiny_qwen2

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('recipe', ['q8', 'q4', 'f16'])
def test_bundle_engine_equals_tensor_engine(gpu_device, tmp_path, recipe):
    print(f'bundle {recipe}', flush=True)
    cfg, w = make_weights(small_cfg(), recipe, seed=5)
    native_bundle.convert(write_bundle(tmp_path / 'hf', cfg, w), tmp_path / 'b.sp')
    a = Qwen2Engine(tmp_path / 'b.sp', max_tokens=16)
    b = Qwen2Engine(config=cfg, tensors=w, max_tokens=16)
    ids = random_prompt(12, cfg['vocab_size'], seed=1)
    la, _ = a.forward(ids, a.new_cache(32), all_logits=True)
    lb, _ = b.forward(ids, b.new_cache(32), all_logits=True)
    assert torch.equal(la, lb)
    assert list(a.generate(ids, max_new_tokens=6)) == list(b.generate(ids, max_new_tokens=6))


@pytest.mark.parametrize('bits', [8, 4])
def test_converted_float_checkpoint_matches_oracle(gpu_device, tmp_path, bits):
    print(f'bundle converted bits={bits}', flush=True)
    tiny_qwen2(tmp_path)
    native_bundle.convert(tmp_path, tmp_path / 'q.sp', bits=bits)
    eng = Qwen2Engine(tmp_path / 'q.sp', max_tokens=16)
    cfg, t = native_bundle.load(tmp_path / 'q.sp')
    ref = RefQwen2(cfg, dequant_all(cfg, t))
    ids = [1, 7, 3, 9, 4, 2, 8]
    lg, _ = eng.forward(ids, eng.new_cache(16), all_logits=True)
    assert max_rel(lg, ref.forward(ids, ref.new_cache(16), all_logits=True)) < 2e-2
