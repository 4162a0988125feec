"""Helpers shared by the GPU parity tests: the tolerance rule and oracle-cache cloning.

Bars: fp16-class logits agree within max |a - b| / max |b| < TOL per row; greedy ids must equal the oracle's wherever
the oracle row's top-2 margin exceeds TOL * max |logit| (a closer race may go either way under fp16 rounding).
"""
import torch

from oracle.qwen_ref import max_rel, top2_margin

TOL = 2e-2


def fp16_rounded(w):
    """The GPU runs float checkpoints with fp16 matrices: the oracle gets the same rounded matrices."""
    return {k: (v.half().float() if v.dim() == 2 else v.float()) for k, v in w.items()}


def check_greedy(tokens, ref_rows, tol=TOL, what=''):
    """Greedy ids vs the oracle rows that produced them (teacher forcing with the GPU's own tokens).  Returns the
    number of steps where the ids agree."""
    same = 0
    for i, (t, row) in enumerate(zip(tokens, ref_rows)):
        r = int(torch.argmax(row))
        if t == r:
            same += 1
        else:
            assert top2_margin(row) <= tol * float(row.abs().max()), f'{what} step {i}: {t} vs oracle {r}'
    return same


def check_rows(gpu_rows, ref_rows, tol=TOL, what=''):
    """Row-wise max-rel of GPU logits vs oracle logits (every row printed, then checked); returns the worst row's
    value."""
    assert gpu_rows.shape == ref_rows.shape, (gpu_rows.shape, ref_rows.shape)
    errs = [max_rel(gpu_rows[i], ref_rows[i]) for i in range(ref_rows.shape[0])]
    print(f'{what} max-rel per row: ' + ' '.join(f'{e:.2e}' for e in errs), flush=True)
    for i, e in enumerate(errs):
        assert e < tol, f'{what} row {i}: max-rel {e:.3e}'
    return max(errs)


def clone_cache(ref, rc, capacity):
    """A copy of oracle cache `rc` (its first rc.length positions) with room for `capacity` positions."""
    c = ref.new_cache(capacity)
    n = rc.length
    for l in range(ref.n_layers):
        c.keys[l][:, :n].copy_(rc.keys[l][:, :n])
        c.values[l][:, :n].copy_(rc.values[l][:, :n])
    c.length = n
    return c
