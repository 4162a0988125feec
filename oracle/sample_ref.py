"""ORACLE (test infrastructure): filtered sampling -- temperature, top-k, top-p -- restated with a full sort.

Semantics of Qwen2Engine.sample (seedplane/qwen_engine.py:146-156) and the native Sampler::distribution / draw
(native/vulkan_decode/sampler.hpp:22-57, 93-97), in the number format the GPU kernel uses:
  z = fp32(l / fp32(T)); order = z descending, ties by ascending index (sampler.hpp:38, the `desc` comparator),
  compared through the 32-bit order key of the float (so -0.0 sorts below +0.0);
  top-k keeps z >= the k-th largest z (ties kept, qwen_engine.py:151-152 / sampler.hpp:26-32);
  mass m_i = trunc(exp(z_i - z_max) * 2^40) as uint64 (float64 exp), sums exact;
  top-p keeps the sorted prefix whose exclusive cumulative mass <= trunc(p * F) (F = kept mass after top-k;
  qwen_engine.py:153-155 `cumsum - probs > top_p` dropped);
  draw: target = min(trunc(u * K), K - 1) over the kept mass K, first sorted token whose inclusive mass exceeds it.
This restatement sorts the whole row (numpy lexsort) where the kernel uses radix selection; nothing else is shared.
"""
import numpy as np

Q = float(2 ** 40)


def order_key(z):
    b = np.asarray(z, dtype=np.float32).view(np.uint32)
    return np.where(b & np.uint32(0x80000000), ~b, b | np.uint32(0x80000000)).astype(np.uint32)


def kept(row, temperature, top_k=0, top_p=1.0):
    """(ids in sorted order, uint64 masses, kept mass K) of the filtered distribution of one logits row."""
    z = (np.asarray(row, dtype=np.float32) / np.float32(temperature)).astype(np.float32)
    V = z.size
    key = order_key(z)
    order = np.lexsort((np.arange(V), -key.astype(np.int64)))
    ks = key[order]
    zmax = np.float64(z[order[0]])
    keep = np.ones(V, dtype=bool)
    if 0 < top_k < V:
        keep = ks >= ks[top_k - 1]
    ids = order[keep]
    m = (np.exp(z[ids].astype(np.float64) - zmax) * Q).astype(np.uint64)
    F = int(m.sum(dtype=np.uint64))
    K = F
    if top_p < 1.0:
        tp = int(np.uint64(float(top_p) * float(np.float64(F))))
        if tp < F:
            c = np.cumsum(m, dtype=np.uint64)
            j = int(np.argmax(c > np.uint64(tp)))
            ids, m, K = ids[:j + 1], m[:j + 1], int(c[j])
    return ids, m, K


def sample_filtered(row, temperature, top_k, top_p, u):
    ids, m, K = kept(row, temperature, top_k, top_p)
    tgt = min(int(np.uint64(float(u) * float(np.float64(K)))), K - 1)
    c = np.cumsum(m, dtype=np.uint64)
    return int(ids[int(np.argmax(c > np.uint64(tgt)))])
