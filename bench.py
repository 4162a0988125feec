#!/usr/bin/env python3
"""Decode throughput of the MI355X Qwen2 decode step (one GPU).

Workload (default): Qwen2-1.5B shape, int8 weights in blocks of 32 along K with one fp16 scale per block (codes
uniform in [-127, 127], scales |N(0, 0.002)|), fp16 KV in a sliding window of 1024 positions, a 3840-token prompt
prefilled K/V-only, then greedy decode at batch 1 -- one step = one token through all 28 layers, the LM head and the
argmax.  Synthetic random-init weights (no checkpoints offline); inputs resident in HBM before the timed region.

Printed JSON line: value = batch-1 decode tok/s; `hbm_frac_step` = algorithmic bytes per token (packed weights + the
KV window read) x tok/s / 8 TB/s; `bs16` = the same model decoding 16 sequences at once; `roofline` = the dominant
kernel (the SwiGLU gate_up GEMV, the largest launch of the step) timed with HIP events on the engine's stream;
`cpu_baseline` = the CPU oracle (fp32, dequantised weights) on a bounded sample of the same workload.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM = 8.0e12
METRIC = 'decode tok/s (bs1, bs16) + % HBM peak, Qwen2-1.5B shape; verify cost/step'


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kv_bytes_per_token(cfg, visible):
    HD = cfg['hidden_size'] // cfg['num_attention_heads']
    return cfg['num_hidden_layers'] * cfg['num_key_value_heads'] * HD * 2 * 2 * visible


def decode_run(eng, caches, first, steps, graph=True):
    import torch
    toks = list(first)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        toks = [int(t) for t in eng.decode(toks, caches, graph=graph)]
    torch.cuda.synchronize()
    return time.perf_counter() - t0, toks


def prefill_all(eng, caches, prompts):
    return eng.prefill(prompts, caches)


def cpu_baseline(cfg, tensors, window, sample_tokens):
    """Oracle decode tok/s on the host cores: fp32 weights dequantised once (4x the int8 bytes), decode-only
    timing after a 16-token prefill, median of 3 runs after one warm-up (experiments/v17/bench_decode.py:21-25)."""
    import torch
    from oracle.qwen_ref import RefQwen2
    from seedplane_amd.synth import random_prompt
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    ref = RefQwen2(cfg, tensors)
    prompt = random_prompt(16, cfg['vocab_size'], seed=1)
    rates = []
    for run in range(4):
        cache = ref.new_cache(16 + sample_tokens + 1)
        logits = ref.forward(prompt, cache, window=window)
        t0 = time.perf_counter()
        for _ in range(sample_tokens):
            tok = ref.greedy(logits[-1])
            logits = ref.forward([tok], cache, window=window)
        dt = time.perf_counter() - t0
        if run:
            rates.append(sample_tokens / dt)
    rates.sort()
    return {'value': round(rates[1], 3), 'unit': 'tok/s', 'cores': cores, 'kind': 'port',
            'sample': f'{sample_tokens} greedy decode tokens after a 16-token prompt, batch 1, same int8 weights '
                      f'dequantised to fp32 (4x the bytes), median of 3 after a warm-up'}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=256)
    ap.add_argument('--warmup', type=int, default=16)
    ap.add_argument('--no-bs16', action='store_true')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--cpu-sample-tokens', type=int, default=6)
    ap.add_argument('--prompt', type=int, default=3840)
    ap.add_argument('--window', type=int, default=1024)
    ap.add_argument('--layers', type=int, default=None, help='(debug) fewer layers; the result is then not the metric')
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({'error': 'this build measures one GPU only: run with --gpus 1 (no multi-GPU path exists)'}))
        sys.exit(2)

    import torch
    from seedplane_amd import _lib
    from seedplane_amd.presets import preset
    from seedplane_amd.qwen_engine import Qwen2Engine
    from seedplane_amd.synth import make_weights, random_prompt

    torch.cuda.set_device(0)
    over = {} if args.layers is None else {'num_hidden_layers': args.layers}
    cfg = preset('qwen2-1.5b', **over)
    t0 = time.perf_counter()
    cfg, w = make_weights(cfg, 'q8', seed=0)
    log(f'weights generated in {time.perf_counter() - t0:.1f}s')
    t0 = time.perf_counter()
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=64)
    log(f'engine loaded in {time.perf_counter() - t0:.1f}s')
    wbytes, _ = eng.weight_bytes()
    W = args.window

    # ---------------------------------------------------------------- batch 1
    eng.reserve(17, eng.slots_for(args.prompt + args.steps + args.warmup + 8, W))
    prompt = random_prompt(args.prompt, cfg['vocab_size'], seed=0)
    cache = eng.new_cache(args.prompt + args.steps + args.warmup + 8, window=W)
    t0 = time.perf_counter()
    first = prefill_all(eng, [cache], [prompt])
    torch.cuda.synchronize()
    log(f'prefill {args.prompt} tokens in {time.perf_counter() - t0:.2f}s')
    _, toks = decode_run(eng, [cache], first, args.warmup)
    dt, toks = decode_run(eng, [cache], toks, args.steps)
    tok_s = args.steps / dt
    visible = min(W, cache.length)
    step_bytes = wbytes + kv_bytes_per_token(cfg, visible)
    log(f'bs1: {tok_s:.1f} tok/s, {dt / args.steps * 1e3:.3f} ms/token, {step_bytes / 1e9:.3f} GB/token')

    # ---------------------------------------------------------------- dominant kernel roofline
    us, gbytes = eng.time_gemv(_lib.SP_T_GATE_UP, layer=0, n_cols=1, iters=200)
    achieved = gbytes / (us * 1e-6) / 1e9
    roofline = {'bound': 'hbm', 'achieved': round(achieved, 1), 'peak': PEAK_HBM / 1e9, 'unit': 'GB/s',
                'frac': round(achieved * 1e9 / PEAK_HBM, 4), 'traffic': None,
                'kernel': 'k_gemv<Q8, 1 m-tile, gate+up pair> (SwiGLU gate_up, 17920x1536 int8 + scales)',
                'bytes_per_launch': gbytes, 'avg_launch_us': round(us, 3)}
    log(f'gate_up GEMV: {us:.2f} us/launch, {achieved:.0f} GB/s')

    # ---------------------------------------------------------------- batch 16
    bs16 = None
    if not args.no_bs16:
        caches = [eng.new_cache(args.prompt + args.steps + args.warmup + 8, window=W) for _ in range(16)]
        prompts = [random_prompt(args.prompt, cfg['vocab_size'], seed=100 + i) for i in range(16)]
        t0 = time.perf_counter()
        first16 = prefill_all(eng, caches, prompts)
        torch.cuda.synchronize()
        log(f'prefill 16 x {args.prompt} tokens in {time.perf_counter() - t0:.2f}s')
        _, t16 = decode_run(eng, caches, first16, args.warmup)
        steps16 = max(16, args.steps // 2)
        dt16, t16 = decode_run(eng, caches, t16, steps16)
        step16_bytes = wbytes + 16 * kv_bytes_per_token(cfg, min(W, caches[0].length))
        bs16 = {'tok_s': round(16 * steps16 / dt16, 1), 'ms_per_step': round(dt16 / steps16 * 1e3, 4),
                'hbm_frac_step': round(step16_bytes * steps16 / dt16 / PEAK_HBM, 4), 'steps': steps16}
        log(f'bs16: {bs16}')

    cpu = None
    if not args.no_cpu_baseline:
        t0 = time.perf_counter()
        cpu = cpu_baseline(cfg, w, W, args.cpu_sample_tokens)
        log(f'cpu baseline {cpu} in {time.perf_counter() - t0:.1f}s')

    out = {'metric': METRIC, 'value': round(tok_s, 2), 'unit': 'tok/s', 'n_gpus': 1, 'steps': args.steps,
           'warmup': args.warmup, 'ms_per_step': round(dt / args.steps * 1e3, 4), 'higher_is_better': True,
           'scaling': 'weak', 'vs_baseline': None, 'dtype': 'int8 weights, fp16 activations/KV, fp32 accumulate',
           'data': 'synthetic (random-init int8 weights, uniform random prompt ids)',
           'config': {'workload': f'Qwen2-1.5B int8 (block 32, fp16 scale) greedy decode, batch 1, window {W}, '
                                  f'prompt {args.prompt}, {args.steps} timed steps',
                      'layers': cfg['num_hidden_layers'], 'hidden': cfg['hidden_size'], 'vocab': cfg['vocab_size'],
                      'window': W, 'prompt': args.prompt},
           'hbm_frac_step': round(step_bytes * tok_s / PEAK_HBM, 4), 'bytes_per_token': step_bytes,
           'bs16': bs16, 'roofline': roofline, 'cpu_baseline': cpu}
    print(json.dumps(out), flush=True)


if __name__ == '__main__':
    main()
