#!/usr/bin/env python3
"""Decode throughput of the MI355X Qwen2 decode step (one GPU) and the cost of speculative tree verification.

Default workload (the `value`): Qwen2-1.5B shape, int8 weights in blocks of 32 along K with one fp16 scale per
block (codes uniform in [-127, 127], scales |N(0, 0.002)|), fp16 KV in a sliding window of 1024 positions, a
3840-token prompt prefilled K/V-only through the engine, then greedy decode at batch 1 -- one step = one token
through all 28 layers (the persistent one-column kernel), the LM head and the argmax.  Synthetic random-init weights
(no checkpoints offline); inputs resident in HBM before the timed region.

The JSON line also carries:
  hbm_frac_step  algorithmic bytes per token (packed weights + the KV window read) x tok/s / 8 TB/s
  bs16           the same model decoding 16 sequences at once (16 x 3840-token prompts)
  verify         tree verification on the same model over a 2048-position prefix: one pass over 1 + 32 nodes
                 (8 branches x 4 tokens) plus the acceptance kernel, divided by one decode step at that prefix
  roofline       the dominant kernel (the persistent step's kernel: every layer of the token, ~95% of the step),
                 HIP-event timed on the engine's stream, with its rocprofv3-measured HBM traffic
  cpu_baseline   the CPU oracle (fp32, dequantised weights) on a bounded sample of the same workload
  latency        per-token latency quantiles with one host synchronisation per token, the decode / draw split of a
                 T > 0 token, and dispatches_per_token (kernels of the recorded step)
  burst16_05b    Qwen2-0.5B fp16, 16 ragged requests x 32 tokens decoded as one batch
  spec           the full speculative loop (0.5B fp16 drafter, 8 x 4 drafts, T 0.8) on the 1.5B int8 target
  batch32_7b     Qwen2-7B int4, batch 32 at 8192 positions of fp16 KV each
                 (each of the three with tok/s, hbm_frac_step and its dominant kernel's launch time and roofline)
The same three run alone as --workload c2 / spec / c5.
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
PEAK_F16 = 2.5e15
METRIC = 'decode tok/s (bs1, bs16) + % HBM peak, Qwen2-1.5B shape; verify cost/step'


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kv_bytes(cfg, visible):
    HD = cfg['hidden_size'] // cfg['num_attention_heads']
    return cfg['num_hidden_layers'] * cfg['num_key_value_heads'] * HD * 2 * 2 * visible


def sync():
    import torch
    torch.cuda.synchronize()


def decode_run(eng, caches, first, steps, graph=True):
    """`steps` greedy steps of every cache, the ids fed back on the GPU and read back in bursts (decode_greedy)."""
    sync()
    t0 = time.perf_counter()
    ids = eng.decode_greedy([int(t) for t in first], caches, steps, graph=graph)
    sync()
    return time.perf_counter() - t0, [seq[-1] for seq in ids]


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


def verify_cost(eng, cfg, prefix=2048, n_branches=8, depth=4, reps=20):
    """Tree verification vs one decode step over the same 2048-position prefix (full attention).  verify_ms: the
    logits pass alone (back-to-back passes); accept_ms: the acceptance walk alone; step_ms: pass + walk timed
    together as a speculative step runs them (the walk waits for the GPU); verify_over_decode = step_ms / decode_ms."""
    import numpy as np
    import torch
    from seedplane_amd.speculative import TreeVerifier, flatten, uniforms
    from seedplane_amd.synth import random_prompt
    V = cfg['vocab_size']
    eng.reserve(1, prefix + 2 * 64 + 64)
    cache = eng.new_cache(prefix + 2 * 64)
    eng.fill_cache(cache, prefix, seed=7)
    rng = np.random.default_rng(0)
    branches = [list(rng.integers(0, V, depth)) for _ in range(n_branches)]
    tree = flatten(int(rng.integers(0, V)), branches)
    verifier = TreeVerifier(eng)
    for _ in range(3):
        p = verifier.forward(cache, tree, graph=True, ids=False)
    sync()
    t0 = time.perf_counter()
    for _ in range(reps):
        p = verifier.forward(cache, tree, graph=True, ids=False)   # logits for the acceptance walk (engine buffer)
    sync()
    t_verify = (time.perf_counter() - t0) / reps
    g = torch.Generator(device=p.device).manual_seed(0)     # a fixed drafter: every run walks the same way
    q = p + 0.3 * torch.randn(p.shape, generator=g, device=p.device)
    u = uniforms(3, 0, 64)
    verifier.accept(p, q, tree, u, 0.8)
    sync()
    t0 = time.perf_counter()
    for i in range(reps):
        verifier.accept(p, q, tree, uniforms(3, i, 64), 0.8)
    sync()
    t_accept = (time.perf_counter() - t0) / reps
    # one speculative step as the loop runs it: the pass, then the acceptance walk (which waits for the GPU)
    t0 = time.perf_counter()
    for i in range(reps):
        p = verifier.forward(cache, tree, graph=True, ids=False)
        verifier.accept(p, q, tree, uniforms(3, i, 64), 0.8)
    sync()
    t_step = (time.perf_counter() - t0) / reps
    tok = int(rng.integers(0, V))
    for _ in range(3):
        eng.decode([tok], [cache], graph=True)
        cache.length = prefix
    sync()
    t0 = time.perf_counter()
    for _ in range(reps):
        eng.decode([tok], [cache], graph=True)
        cache.length = prefix                    # roll back: every step at the same prefix
    sync()
    t_decode = (time.perf_counter() - t0) / reps
    wbytes, _ = eng.weight_bytes()
    flops = 2.0 * (wbytes / 1.0625) * tree.size      # ~params x columns (int8 + fp16 scale per 32 = 1.0625 B/param)
    return {'nodes': tree.size, 'prefix': prefix, 'verify_ms': round(t_verify * 1e3, 4),
            'accept_ms': round(t_accept * 1e3, 4), 'step_ms': round(t_step * 1e3, 4),
            'decode_ms': round(t_decode * 1e3, 4),
            'verify_over_decode': round(t_step / t_decode, 3),
            'verify_pass_over_decode': round(t_verify / t_decode, 3),
            'verify_tflops': round(flops / t_verify / 1e12, 2),
            'mfma_frac_f16': round(flops / t_verify / PEAK_F16, 4)}


def sampling_cost(eng, V, rows=16, reps=20):
    """GPU filtered draws (temperature 0.8, top-k / top-p) over `rows` fp32 logits rows of the full vocabulary:
    microseconds per launch of `rows` draws (HIP events on the launching stream) and per draw, for each filter."""
    import numpy as np
    import torch
    from seedplane_amd.speculative import uniforms
    g = torch.Generator(device='cuda').manual_seed(0)
    lg = torch.randn((rows, V), generator=g, device='cuda') * 3.0
    rid = torch.arange(rows, dtype=torch.int32, device='cuda')
    res = {}
    for name, k, p in (('top_k50_top_p0.9', 50, 0.9), ('top_p0.9', 0, 0.9), ('temperature_only', 0, 1.0)):
        u = uniforms(1, 0, rows)
        eng.sample_gpu(lg, None, u, 0.8, k, p, rows_dev=rid)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        sync()
        e0.record()
        for i in range(reps):
            eng.sample_gpu(lg, None, uniforms(1, i, rows), 0.8, k, p, rows_dev=rid)
        e1.record()
        sync()
        us = e0.elapsed_time(e1) * 1e3 / reps
        res[name] = {'us_per_launch': round(us, 1), 'draws_per_launch': rows}
    return res


TRAFFIC_FILE = ROOT / 'profiles' / 'k_decode1_q8_15b_bs1_traffic.md'
KERNEL_SOURCES = ('sp_decode1.h', 'sp_gemv.h', 'sp_attn.h', 'sp_device.h', 'sp_pack.h')


def kernel_source_hash():
    """First 16 hex digits of the SHA-256 over the persistent kernel's sources (kernel, GEMV tiles, attention and
    device helpers, tile packing)."""
    import hashlib
    h = hashlib.sha256()
    for name in KERNEL_SOURCES:
        h.update((ROOT / 'seedplane_amd' / 'csrc' / name).read_bytes())
    return h.hexdigest()[:16]


def measured_traffic():
    """HBM bytes per persistent-kernel launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (each
    counter scaled by what it reads for a plain copy of known size), and whether it applies: the summary records the
    hash of the kernel sources it was measured on, and a summary of other sources is reported as stale (traffic
    null)."""
    fields = {}
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            if ':' in line and line.split(':')[0] in ('traffic_bytes_per_launch', 'kernel_source_sha16'):
                k, v = line.split(':', 1)
                fields[k] = v.strip()
    except OSError:
        return None, 'no traffic summary'
    if 'traffic_bytes_per_launch' not in fields:
        return None, 'no traffic summary'
    if fields.get('kernel_source_sha16') != kernel_source_hash():
        return None, 'traffic summary measured on other kernel sources (stale)'
    return int(fields['traffic_bytes_per_launch']), f'{TRAFFIC_FILE.relative_to(ROOT)} (rocprofv3 --pmc, scaled)'


def token_latency(eng, cache, token, n=64, warm=4):
    """Per-token latency as a caller sees it that needs each id before the next step (one host synchronisation per
    token, the reference's session loop, native/vulkan_decode/qwen_vk.cpp:883-897): quantiles over n tokens, the
    kernels one step launches (the recorded step's kernel nodes), and the split of a T > 0 token into the decode step
    and the GPU draw (top-k 50 / top-p 0.9 at T = 0.8 over the step's logits row, HIP events)."""
    import torch
    from seedplane_amd.speculative import uniforms
    lat = []
    for i in range(n + warm):
        t0 = time.perf_counter()
        token = int(eng.decode([token], [cache], graph=True)[0])
        if i >= warm:
            lat.append(time.perf_counter() - t0)
    dispatches = eng.last_dispatches
    row = torch.empty((1, eng.vocab), dtype=torch.float32, device=eng.device)
    eng.decode([token], [cache], logits_out=row, graph=True)
    rid = torch.zeros(1, dtype=torch.int32, device=eng.device)
    eng.sample_gpu(row, None, uniforms(2, 0, 1), 0.8, 50, 0.9, rows_dev=rid)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    sync()
    e0.record()
    for i in range(20):
        eng.sample_gpu(row, None, uniforms(2, i, 1), 0.8, 50, 0.9, rows_dev=rid)
    e1.record()
    sync()
    srt = sorted(lat)
    q = lambda f: round(1e3 * srt[min(len(srt) - 1, int(f * (len(srt) - 1) + 0.5))], 4)
    return {'p50_ms': q(0.5), 'p95_ms': q(0.95), 'p99_ms': q(0.99), 'max_ms': round(1e3 * srt[-1], 4),
            'step_ms_mean': round(1e3 * sum(lat) / len(lat), 4), 'sample_ms_mean': round(e0.elapsed_time(e1) / 20, 4),
            'tokens': n, 'sync': 'one host synchronisation per token'}, dispatches


def kernel_frac(name, us, nbytes):
    """A dominant kernel's measured launch time and its fraction of the HBM roofline for its algorithmic bytes."""
    return {'kernel': name, 'avg_launch_us': round(us, 3), 'bytes_per_launch': nbytes,
            'achieved_gbs': round(nbytes / (us * 1e-6) / 1e9, 1), 'frac': round(nbytes / (us * 1e-6) / PEAK_HBM, 4)}


def step_roofline(eng, cache, iters=50):
    """The dominant kernel: the persistent one-column step's kernel (every layer of one token), launched for a
    decode column of `cache` on the engine's stream, HIP-event timed there.  Algorithmic bytes per launch: all 28
    layers' int8 codes and fp16 scales, norm weights and qkv bias, the window's K and V, the embedding row."""
    us, nbytes = eng.time_persistent(cache, iters=iters)
    achieved = nbytes / (us * 1e-6) / 1e9
    log(f'persistent step kernel: {us:.2f} us/launch, {nbytes} bytes, {achieved:.0f} GB/s')
    traffic, source = measured_traffic()
    return {'bound': 'hbm', 'achieved': round(achieved, 1), 'peak': PEAK_HBM / 1e9, 'unit': 'GB/s',
            'frac': round(achieved * 1e9 / PEAK_HBM, 4), 'traffic': traffic, 'traffic_source': source,
            'kernel': 'd1::k_decode1<Q8, head_dim 128> (persistent one-column step: 28 layers of Qwen2-1.5B int8, '
                      'one block per CU)',
            'bytes_per_launch': nbytes, 'avg_launch_us': round(us, 3)}


def workload_roofline(args, out):
    """Only the dominant kernel's timing (for counter runs: 51 launches of the persistent kernel at 1100 cached
    positions, window 1024), then a plain 512 MiB copy (torch elementwise multiply by 1.0) whose FETCH_SIZE /
    WRITE_SIZE give the counters' scale."""
    import torch
    from seedplane_amd.presets import preset
    from seedplane_amd.qwen_engine import Qwen2Engine
    from seedplane_amd.synth import make_weights, random_prompt
    cfg, w = make_weights(preset('qwen2-1.5b'), 'q8', seed=0)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=64)
    cache = eng.new_cache(4096, window=args.window)
    eng.prefill([random_prompt(1100, cfg['vocab_size'], seed=1)], [cache])
    out['roofline'] = step_roofline(eng, cache)
    src = torch.ones(128 << 20, dtype=torch.float32, device='cuda')
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    sync()
    out.update({'value': out['roofline']['achieved'], 'unit': 'GB/s', 'metric': 'persistent step kernel HBM GB/s',
                'copy_bytes_each_way': src.numel() * 4})


def workload_c3(args, out):
    import torch
    from seedplane_amd import _lib
    from seedplane_amd.presets import preset
    from seedplane_amd.qwen_engine import Qwen2Engine
    from seedplane_amd.synth import make_weights, random_prompt
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
    cap = args.prompt + args.steps + args.warmup + 8
    eng.reserve(17, eng.slots_for(cap, W))
    prompt = random_prompt(args.prompt, cfg['vocab_size'], seed=0)
    cache = eng.new_cache(cap, window=W)
    t0 = time.perf_counter()
    first = eng.prefill([prompt], [cache])
    sync()
    log(f'prefill {args.prompt} tokens in {time.perf_counter() - t0:.2f}s')
    _, toks = decode_run(eng, [cache], first, args.warmup)
    dt, toks = decode_run(eng, [cache], toks, args.steps)
    tok_s = args.steps / dt
    step_bytes = wbytes + kv_bytes(cfg, min(W, cache.length))
    log(f'bs1: {tok_s:.1f} tok/s, {dt / args.steps * 1e3:.3f} ms/token, {step_bytes / 1e9:.3f} GB/token')
    latency, dispatches = token_latency(eng, cache, toks[0])
    log(f'latency: {latency}, {dispatches} kernels per step')

    roofline = step_roofline(eng, cache)

    bs16 = None
    if not args.no_bs16:
        caches = [eng.new_cache(cap, window=W) for _ in range(16)]
        prompts = [random_prompt(args.prompt, cfg['vocab_size'], seed=100 + i) for i in range(16)]
        t0 = time.perf_counter()
        first16 = eng.prefill(prompts, caches)
        sync()
        log(f'prefill 16 x {args.prompt} tokens in {time.perf_counter() - t0:.2f}s')
        _, t16 = decode_run(eng, caches, first16, args.warmup)
        steps16 = max(16, args.steps // 2)
        dt16, t16 = decode_run(eng, caches, t16, steps16)
        b16 = wbytes + 16 * kv_bytes(cfg, min(W, caches[0].length))
        bs16 = {'tok_s': round(16 * steps16 / dt16, 1), 'ms_per_step': round(dt16 / steps16 * 1e3, 4),
                'hbm_frac_step': round(b16 * steps16 / dt16 / PEAK_HBM, 4), 'steps': steps16}
        log(f'bs16: {bs16}')

    verify = None
    if not args.no_verify:
        verify = verify_cost(eng, cfg)
        log(f'verify: {verify}')

    sampling = sampling_cost(eng, cfg['vocab_size'])
    log(f'sampling: {sampling}')

    extra = {}
    if not args.no_extra:
        extra['burst16_05b'], drafter = run_c2(return_engine=True)
        log(f"burst16_05b: {extra['burst16_05b']}")
        extra['spec'] = run_spec(eng, cfg, drafter)
        log(f"spec: {extra['spec']}")
        del drafter
        extra['batch32_7b'] = run_c5(128)
        log(f"batch32_7b: {extra['batch32_7b']}")

    cpu = None
    if not args.no_cpu_baseline:
        t0 = time.perf_counter()
        cpu = cpu_baseline(cfg, w, W, args.cpu_sample_tokens)
        log(f'cpu baseline {cpu} in {time.perf_counter() - t0:.1f}s')

    out.update({'metric': METRIC, 'value': round(tok_s, 2), 'unit': 'tok/s', 'steps': args.steps,
                'warmup': args.warmup, 'ms_per_step': round(dt / args.steps * 1e3, 4), 'higher_is_better': True,
                'dtype': 'int8 weights, fp16 activations/KV, fp32 accumulate',
                'data': 'synthetic (random-init int8 weights, uniform random prompt ids)',
                'config': {'workload': f'Qwen2-1.5B int8 (block 32, fp16 scale) greedy decode, batch 1, window {W}, '
                                       f'prompt {args.prompt}, {args.steps} timed steps',
                           'layers': cfg['num_hidden_layers'], 'hidden': cfg['hidden_size'],
                           'vocab': cfg['vocab_size'], 'window': W, 'prompt': args.prompt},
                'hbm_frac_step': round(step_bytes * tok_s / PEAK_HBM, 4), 'bytes_per_token': step_bytes,
                'latency': latency, 'dispatches_per_token': dispatches,
                'bs16': bs16, 'verify': verify, 'sampling': sampling, **extra, 'roofline': roofline,
                'cpu_baseline': cpu})


def workload_verify(args, out):
    """Only the tree-verification cost on the 1.5B int8 model (for profiling)."""
    from seedplane_amd.presets import preset
    from seedplane_amd.qwen_engine import Qwen2Engine
    from seedplane_amd.synth import make_weights
    cfg, w = make_weights(preset('qwen2-1.5b'), 'q8', seed=0)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=64)
    v = verify_cost(eng, cfg)
    out.update({'metric': 'tree verify cost / decode step (1 + 8x4 nodes, 2048 prefix)',
                'value': v['verify_over_decode'], 'unit': 'ratio', 'higher_is_better': False, 'verify': v})


def run_c2(return_engine=False):
    """Qwen2-0.5B fp16, 16 requests x 32 greedy tokens, prompts of 16-128 ids, decoded as one batch (decode-only
    timing; the K/V-only prefill is outside it).  Dominant kernel: the 16-column SwiGLU gate_up GEMV."""
    import torch
    from seedplane_amd import _lib
    from seedplane_amd.presets import preset
    from seedplane_amd.qwen_engine import Qwen2Engine
    from seedplane_amd.synth import make_weights, random_prompt
    cfg, w = make_weights(preset('qwen2-0.5b'), 'f16', seed=0)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=64)
    del w
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(16, 129, (16,), generator=g).tolist()
    prompts = [random_prompt(n, cfg['vocab_size'], seed=200 + i) for i, n in enumerate(lens)]
    new = 32
    eng.reserve(16, 512)
    caches = [eng.new_cache(512) for _ in range(16)]
    first = eng.prefill(prompts, caches)
    dt, _ = decode_run(eng, caches, first, new - 1)
    tok_s = 16 * (new - 1) / dt
    wbytes, _ = eng.weight_bytes()
    mean_ctx = sum(c.length for c in caches) / 16
    step_bytes = wbytes + 16 * kv_bytes(cfg, mean_ctx)
    us, nb = eng.time_gemv(_lib.SP_T_GATE_UP, layer=-1, n_cols=16, iters=240)
    res = {'workload': 'Qwen2-0.5B fp16, 16 requests x 32 greedy tokens, prompts of 16-128 ids, batch 16',
           'tok_s': round(tok_s, 1), 'ms_per_step': round(dt / (new - 1) * 1e3, 4),
           'hbm_frac_step': round(step_bytes * (new - 1) / dt / PEAK_HBM, 4), 'prompt_lens': lens,
           'dominant_kernel': kernel_frac('k_gemv<F16, 1 m-tile, gate+up pair> 16 columns (9728x896 fp16)', us, nb)}
    return (res, eng) if return_engine else res


def run_c5(steps=128):
    """Qwen2-7B int4 (g32 scale + zero), batch 32 at 8192 positions of full fp16 KV each.  The 8192-token contexts are
    filled with seeded synthetic K/V (the decode step reads the same bytes).  Dominant kernel: the MFMA decode attention
    (the K/V of 32 x 8192 positions is 77% of a step's bytes)."""
    from seedplane_amd.presets import preset
    from seedplane_amd.qwen_engine import Qwen2Engine
    from seedplane_amd.synth import make_weights, random_prompt
    t0 = time.perf_counter()
    cfg, w = make_weights(preset('qwen2-7b'), 'q4', seed=0)
    log(f'7B int4 weights generated in {time.perf_counter() - t0:.1f}s')
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=64)
    del w
    ctx, B = 8192, 32
    eng.reserve(B, ctx + steps + 8)
    caches = [eng.new_cache(ctx + steps + 8) for _ in range(B)]
    for i, c in enumerate(caches):
        eng.fill_cache(c, ctx, seed=i)
    toks = random_prompt(B, cfg['vocab_size'], seed=5)
    _, toks = decode_run(eng, caches, toks, 4)
    dt, _ = decode_run(eng, caches, toks, steps)
    tok_s = B * steps / dt
    wbytes, _ = eng.weight_bytes()
    step_bytes = wbytes + B * kv_bytes(cfg, ctx + steps // 2)
    us, nb = eng.time_attention(caches, iters=56)
    return {'workload': 'Qwen2-7B int4, batch 32, 8192-token full fp16 KV per request',
            'tok_s': round(tok_s, 1), 'ms_per_step': round(dt / steps * 1e3, 4), 'steps': steps,
            'hbm_frac_step': round(step_bytes * steps / dt / PEAK_HBM, 4), 'bytes_per_step': step_bytes,
            'dominant_kernel': kernel_frac('k_attn_dec<128> (32 x ~8260 keys, 4 kv heads, GQA 7)', us, nb)}


def run_spec(target, cfg, drafter_engine, steps=32):
    """The full speculative loop: target 1.5B int8, drafter 0.5B fp16, 8 branches x 4 tokens, T = 0.8, seeded
    uniforms, over a 2048-token prompt; both models' prefills run before the timed steps.  Random-init models are
    unrelated, so few drafts are accepted; the figure is the cost of a step, not a speedup.
    budget: the parts of a step timed alone, each call followed by a synchronisation -- the drafter's root pass (one
    column), one drafter level (8 tree columns over the 24-node draft tree), the target's verify step (the 33-node
    pass + the acceptance walk) -- and budget_ms = root + 3 levels + verify step + 0.3 ms, against ms_per_step."""
    import numpy as np
    import torch
    from seedplane_amd import _lib
    from seedplane_amd.speculative import SpecStats, SpeculativeLoop, TreeDrafter, TreeVerifier, flatten, uniforms
    from seedplane_amd.synth import random_prompt
    drafter = TreeDrafter(drafter_engine)
    prompt = random_prompt(2048, cfg['vocab_size'], seed=9)
    warm = SpeculativeLoop(target, drafter, prompt, seed=0, capacity=len(prompt) + 64)
    for _ in range(2):
        warm.step()
    del warm
    stats = SpecStats()
    loop = SpeculativeLoop(target, drafter, prompt, seed=1, stats=stats, capacity=len(prompt) + 5 * steps + 128)
    sync()
    t0 = time.perf_counter()
    toks = []
    for _ in range(steps):
        toks += loop.step()
    sync()
    dt = time.perf_counter() - t0

    def alone(fn, reps=20):
        fn()
        sync()
        t = time.perf_counter()
        for _ in range(reps):
            fn()
            sync()
        return (time.perf_counter() - t) / reps * 1e3
    dc, tc, tok = loop.dcache, loop.tcache, loop.committed[-1]

    def root():
        drafter_engine.forward([tok], dc)
        dc.length -= 1
    L, S = dc.length, drafter_engine._pool_slots
    cols = [(5 + b, dc.seq, L + 2, (L + 16 + b) % S, 0, L - 1, L % S, 24,       # level 3 of the draft tree
             (1 << b) | (1 << (8 + b)) | (1 << (16 + b))) for b in range(8)]
    lout = torch.empty((8, drafter_engine.vocab), dtype=torch.float32, device=drafter_engine.device)
    rng = np.random.default_rng(0)
    tree = flatten(tok, [list(rng.integers(0, cfg['vocab_size'], 4)) for _ in range(8)])
    verifier = TreeVerifier(target)
    p = verifier.forward(tc, tree, ids=False)
    g = torch.Generator(device=p.device).manual_seed(0)
    q = p + 0.3 * torch.randn(p.shape, generator=g, device=p.device)
    u = uniforms(3, 0, 64)

    def verify_step():
        pp = verifier.forward(tc, tree, ids=False)
        verifier.accept(pp, q, tree, u, 0.8)
    root_ms = alone(root)
    level_ms = alone(lambda: drafter_engine.run(cols, _lib.SP_F_LOGITS, logits_out=lout))
    verify_ms = alone(verify_step)
    budget = root_ms + 3 * level_ms + verify_ms + 0.3
    us, nb = target.time_gemv(_lib.SP_T_GATE_UP, layer=-1, n_cols=33, iters=140)
    return {'workload': 'target Qwen2-1.5B int8, drafter Qwen2-0.5B fp16, 8 branches x 4, T 0.8, 2048-token prompt',
            'tok_s': round(len(toks) / dt, 2), 'ms_per_step': round(dt / steps * 1e3, 3), 'steps': steps,
            'accepted_per_step': round(stats.accepted / stats.steps, 3),
            'emitted_per_step': round(stats.emitted / stats.steps, 3),
            'budget': {'drafter_root_ms': round(root_ms, 3), 'drafter_level_ms': round(level_ms, 3),
                       'verify_step_ms': round(verify_ms, 3), 'budget_ms': round(budget, 3),
                       'step_within_budget': dt / steps * 1e3 <= budget},
            'dominant_kernel': kernel_frac('k_gemv<Q8, 3 m-tiles, gate+up pair> 33 columns (tree pass)', us, nb)}


def workload_c2(args, out):
    r = run_c2()
    out.update({'metric': 'decode tok/s, 16-request burst, Qwen2-0.5B fp16', 'value': r['tok_s'], 'unit': 'tok/s',
                'steps': 31, 'warmup': 0, 'ms_per_step': r['ms_per_step'], 'higher_is_better': True,
                'dtype': 'fp16 weights/activations/KV, fp32 accumulate',
                'data': 'synthetic (random-init fp16 weights ~N(0,0.02), uniform random prompts of 16-128 ids)',
                'config': {'workload': r['workload'], 'prompt_lens': r['prompt_lens']},
                'hbm_frac_step': r['hbm_frac_step'], 'dominant_kernel': r['dominant_kernel']})


def workload_c5(args, out):
    steps = args.steps if args.steps != 256 else 128
    r = run_c5(steps)
    out.update({'metric': 'decode tok/s, Qwen2-7B int4 batch 32 at 8k context', 'value': r['tok_s'], 'unit': 'tok/s',
                'steps': steps, 'warmup': 4, 'ms_per_step': r['ms_per_step'], 'higher_is_better': True,
                'dtype': 'int4 weights (g32 fp16 scale+zero), fp16 activations/KV',
                'data': 'synthetic (random-init int4 weights; 8192-position contexts filled with seeded K/V)',
                'config': {'workload': r['workload']}, 'hbm_frac_step': r['hbm_frac_step'],
                'bytes_per_step': r['bytes_per_step'], 'dominant_kernel': r['dominant_kernel']})


def workload_spec(args, out):
    from seedplane_amd.presets import preset
    from seedplane_amd.qwen_engine import Qwen2Engine
    from seedplane_amd.synth import make_weights
    cfg, w = make_weights(preset('qwen2-1.5b'), 'q8', seed=0)
    target = Qwen2Engine(config=cfg, tensors=w, max_tokens=64)
    dcfg, dw = make_weights(preset('qwen2-0.5b'), 'f16', seed=1)
    r = run_spec(target, cfg, Qwen2Engine(config=dcfg, tensors=dw, max_tokens=64), steps=64)
    out.update({'metric': 'speculative tree decode tok/s (8x4 drafts, T=0.8)', 'value': r['tok_s'], 'unit': 'tok/s',
                'steps': 64, 'warmup': 2, 'ms_per_step': r['ms_per_step'], 'higher_is_better': True,
                'dtype': 'target int8 / drafter fp16, fp32 logits, fp64 acceptance',
                'data': 'synthetic random-init target and drafter (acceptance is near zero for unrelated models)',
                'config': {'workload': r['workload']},
                **{k: r[k] for k in ('accepted_per_step', 'emitted_per_step', 'budget')}})


def workload_sampling(args, out):
    """The filtered sampler alone: 16 draws per launch over 16 rows of 151936 fp32 logits (the Qwen2 vocabulary),
    T = 0.8, for three filters.  The draws use only the library's sampling op; a tiny engine provides the handle."""
    from seedplane_amd.presets import preset
    from seedplane_amd.qwen_engine import Qwen2Engine
    from seedplane_amd.synth import make_weights
    cfg, w = make_weights(preset('tiny'), 'q8', seed=0)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=16)
    r = sampling_cost(eng, 151936, reps=20)
    main_us = r['top_k50_top_p0.9']['us_per_launch']
    out.update({'metric': 'filtered sampling launch time (16 draws, top-k 50 + top-p 0.9, T 0.8)', 'value': main_us,
                'unit': 'us/launch', 'steps': 20, 'warmup': 1, 'ms_per_step': round(main_us / 1e3, 4),
                'higher_is_better': False, 'dtype': 'fp32 logits, 64-bit integer masses',
                'data': 'synthetic (N(0, 3) logits, seeded uniforms)',
                'config': {'workload': '16 rows x 151936 fp32 logits, one draw per row'}, 'sampling': r})


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=256)
    ap.add_argument('--warmup', type=int, default=16)
    ap.add_argument('--workload', default='c3', choices=['c3', 'c2', 'c5', 'spec', 'verify', 'roofline', 'sampling'])
    ap.add_argument('--no-bs16', action='store_true')
    ap.add_argument('--no-verify', action='store_true')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--no-extra', action='store_true', help='skip the 0.5B burst, speculative loop and 7B int4 lines')
    ap.add_argument('--cpu-sample-tokens', type=int, default=6)
    ap.add_argument('--prompt', type=int, default=3840)
    ap.add_argument('--window', type=int, default=1024)
    ap.add_argument('--layers', type=int, default=None, help='(debug) fewer layers; the result is then not the metric')
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({'error': 'this build measures one GPU only: run with --gpus 1 (no multi-GPU path exists)'}))
        sys.exit(2)
    import torch
    torch.cuda.set_device(0)
    out = {'metric': METRIC, 'value': None, 'unit': 'tok/s', 'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup,
           'ms_per_step': None, 'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None}
    {'c3': workload_c3, 'c2': workload_c2, 'c5': workload_c5, 'spec': workload_spec, 'verify': workload_verify,
     'roofline': workload_roofline, 'sampling': workload_sampling}[args.workload](args, out)
    print(json.dumps(out), flush=True)


if __name__ == '__main__':
    main()
