"""ORACLE (test infrastructure): speculative-decoding semantics restated on the CPU.

  * Forest / verify_greedy / ledger: seedplane/speculative.py:12-111 (same decisions, same tie rules).
  * Linear batched verify with rollback: experiments/hive_scaling/benchmark_speculative.py:59-135.
  * Seeded uniforms: SplitMix64 (Steele, Lea, Flood 2014) over a counter, u = (x >> 11) * 2^-53.
  * Float64 draws and tree acceptance in the product's fixed summation orders (draw: 1024 contiguous chunks, each
    summed in index order, chunk sums added in chunk order; accept_tree / draw3: 64 x 256 chunks, summed per chunk,
    per group of 256 by wave butterflies, then over groups), so decisions can be compared bit for bit; each function
    also returns the smallest decision margin so a test can show no comparison was within rounding of its threshold.
  * Pins: draw / draw3 against a brute-force inverse CDF in exact rational arithmetic (zeros, single positive
    entries, top-of-range targets); accept_tree through the speculative sampling theorem (Monte Carlo over the
    uniform-driven walk) and through per-trial thresholds recomputed with the iterative residual definition.
  * exact_first_token_distribution: the acceptance rule's output law computed analytically over every draft outcome
    (speculative sampling theorem: it must equal the target distribution p).
"""
from dataclasses import dataclass, field
from itertools import product

import numpy as np

NCHUNK = 1024
MASK64 = (1 << 64) - 1


# ------------------------------------------------------------------------------------------- reference semantics
@dataclass
class Node:
    token: int
    children: dict = field(default_factory=dict)


@dataclass
class Forest:
    roots: dict = field(default_factory=dict)
    paths: list = field(default_factory=list)

    @classmethod
    def build(cls, branches):
        """speculative.py:24-37: non-empty branches kept in input order; shared prefixes share nodes."""
        f = cls()
        for branch in branches:
            path = tuple(int(t) for t in branch)
            if not path:
                continue
            f.paths.append(path)
            level = f.roots
            for t in path:
                if t not in level:
                    level[t] = Node(t)
                level = level[t].children
        return f

    def node_count(self):
        def count(level):
            return sum(1 + count(n.children) for n in level.values())
        return count(self.roots)


def first_argmax(values):
    """Python's max(range(n), key=...) picks the first maximal index (speculative.py:68,80)."""
    best = 0
    for i in range(1, len(values)):
        if values[i] > values[best]:
            best = i
    return best


def verify_greedy(committed, forest, target_logits):
    """speculative.py:55-92."""
    base = tuple(int(t) for t in committed)
    if not forest.paths:
        logits = target_logits(base)
        if not len(logits):
            raise ValueError('target returned empty logits')
        return ((first_argmax(logits),), 0, False, 1, ())
    best = None
    for path in forest.paths:
        accepted, steps, rejected = [], 0, False
        for draft in path:
            logits = target_logits(base + tuple(accepted))
            tok = first_argmax(logits)
            steps += 1
            if draft != tok:
                accepted.append(tok)
                rejected = True
                break
            accepted.append(draft)
        res = (tuple(accepted), len(accepted) - int(rejected), rejected, steps, path)
        if best is None or (res[1], len(res[0])) > (best[1], len(best[0])):
            best = res
    return best


def linear_verify(draft, pre_logits_argmax, block_argmax):
    """benchmark_speculative.py:85-131: draft[0] against the pre-wave argmax, draft[i] against row i-1 of the
    batched pass; returns (emitted tokens, accepted count, rolled-back cache length offset)."""
    if draft[0] != pre_logits_argmax:
        return [pre_logits_argmax], 0, 0
    accepted = 1
    for i in range(1, len(draft)):
        if draft[i] != block_argmax[i - 1]:
            return list(draft[:accepted]) + [block_argmax[i - 1]], accepted, accepted
        accepted += 1
    return list(draft), accepted, accepted


# ------------------------------------------------------------------------------------------- uniforms
def splitmix64(x):
    x = (x + 0x9E3779B97F4A7C15) & MASK64
    z = x
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def uniforms(seed, step, n):
    """u_i = (splitmix64(splitmix64(seed) ^ (step * 2^20 + i)) >> 11) * 2^-53, i < n."""
    s = splitmix64(seed & MASK64)
    return np.array([(splitmix64(s ^ ((step << 20) + i)) >> 11) * 2.0 ** -53 for i in range(n)], dtype=np.float64)


# ------------------------------------------------------------------------------------------- fixed-order float64
def softmax_weights(logits, temperature):
    l = np.asarray(logits, dtype=np.float32)
    m = np.float64(l.max())
    inv_t = 1.0 / float(temperature)
    return np.exp((l.astype(np.float64) - m) * inv_t)


def chunk_sums(w):
    """Per-chunk sequential sums (np.cumsum is sequential) and their sequential total."""
    V = len(w)
    C = -(-V // NCHUNK)
    padded = np.zeros(NCHUNK * C)
    padded[:V] = w
    sums = np.cumsum(padded.reshape(NCHUNK, C), axis=1)[:, -1]
    total = np.cumsum(sums)[-1]
    return sums, total, C


def draw(w, u):
    """Inverse CDF with the chunked order.  Returns (token, margin) where margin is the smallest relative gap
    between the target and a compared running sum / chunk boundary."""
    sums, total, C = chunk_sums(w)
    prefix = np.concatenate([[0.0], np.cumsum(sums)[:-1]])
    target = u * total
    upper = np.append(target < prefix[1:], True)
    t_sel = int(np.flatnonzero((target >= prefix) & upper)[0])
    pos = prefix[1:][prefix[1:] > 0]
    margin = float(np.min(np.abs(target - pos)) / total) if len(pos) else np.inf
    V = len(w)
    lo, hi = t_sel * C, min(V, (t_sel + 1) * C)
    tl = target - prefix[t_sel]
    acc, pick, lastpos = 0.0, -1, -1
    for i in range(lo, hi):
        if w[i] > 0:
            lastpos = i
        acc += w[i]
        margin = min(margin, abs(acc - tl) / total)
        if acc > tl:
            pick = i
            break
    if pick < 0:
        pick = lastpos
    if pick < 0:
        pick = V - 1
        while pick > 0 and not w[pick] > 0:
            pick -= 1
    return int(pick), margin


ACC_NB, ACC_T = 64, 256


def _butterfly(v):
    """Sum of 64 values the way a wave's xor butterfly takes it (lane l adds lane l ^ o, o = 32, 16, ..., 1)."""
    v = v.copy()
    lanes = np.arange(64)
    for o in (32, 16, 8, 4, 2, 1):
        v = v + v[..., lanes ^ o]
    return v[..., 0]


def chunk_sums3(w):
    """Acceptance-walk summation order: ACC_NB * ACC_T contiguous chunks of C = ceil(V / (ACC_NB * ACC_T)) entries,
    each summed in index order; each group of ACC_T chunk sums reduced by a butterfly inside every 64-lane wave,
    the wave sums added in order; the ACC_NB group sums added in order.  Returns (chunk sums, group sums, total, C)."""
    V = len(w)
    G = ACC_NB * ACC_T
    C = -(-V // G)
    padded = np.zeros(G * C)
    padded[:V] = w
    tsum = np.cumsum(padded.reshape(G, C), axis=1)[:, -1]
    wsum = _butterfly(tsum.reshape(ACC_NB, ACC_T // 64, 64))
    bsum = np.cumsum(wsum, axis=1)[:, -1]
    return tsum, bsum, np.cumsum(bsum)[-1], C


def _first_exceeding(parts, target):
    """Index of the first entry whose running sum exceeds target, else the last positive entry (0 if none), the
    running sum before it, and the smallest |target - running sum| over the compared positive entries."""
    run, last, run_last, gap = 0.0, 0, 0.0, np.inf
    for i, v in enumerate(parts):
        nxt = run + v
        if v > 0:
            last, run_last = i, run
            gap = min(gap, abs(target - nxt))
        if target < nxt:
            return i, run, gap
        run = nxt
    return last, run_last, gap


def block_weights(logits, temperature):
    """Acceptance-walk weights of one row: group g (ACC_T consecutive chunks) takes its maximum m_g, its entries'
    local weights e_i = exp((l_i - m_g) * (1/T)) (all 0 when m_g = -inf) and their sum s_g in chunk_sums3 order; with
    M the row maximum, f_g = exp((m_g - M) * (1/T)), the normaliser Z is the sum of the partials s_g * f_g in group
    order.  Returns (e, f per entry, partials, Z)."""
    l = np.asarray(logits, dtype=np.float32)
    V = len(l)
    G = ACC_NB * ACC_T
    C = -(-V // G)
    padded = np.full(G * C, -np.inf, dtype=np.float32)
    padded[:V] = l
    m = padded.reshape(ACC_NB, ACC_T * C).max(axis=1).astype(np.float64)
    inv_t = 1.0 / float(temperature)
    mm = np.repeat(m, ACC_T * C)[:V]
    live = mm > -np.inf
    with np.errstate(invalid='ignore'):
        e = np.where(live, np.exp((l.astype(np.float64) - mm) * inv_t), 0.0)
    f = np.exp((m - m.max()) * inv_t)
    parts = chunk_sums3(e)[1] * f
    return e, np.repeat(f, ACC_T * C)[:V], parts, np.cumsum(parts)[-1]


def walk_probs(logits, temperature):
    """p_i = e_i * (f_g / Z), the acceptance walk's probabilities (block_weights)."""
    e, f, _, Z = block_weights(logits, temperature)
    return e * (f / Z)


def draw3(w, u, bsum=None):
    """Inverse CDF over the acceptance-walk chunk tree (group, chunk, element), with its fallbacks: a level whose
    running sums never exceed the target (rounding) takes its last positive entry; with no positive weight at all
    the token is 0.  bsum: group partials to use instead of the sums of w's chunks (a bonus draw takes
    block_weights' partials).  Returns (token, margin) with margin the smallest relative gap at a compared boundary."""
    tsum, own, total, C = chunk_sums3(w)
    if bsum is None:
        bsum = own
    else:
        total = np.cumsum(bsum)[-1]
    V = len(w)
    target = u * total
    scale = total if total > 0 else 1.0
    b, Pb, g1 = _first_exceeding(bsum, target)
    tb = target - Pb
    t, Pt, g2 = _first_exceeding(tsum[b * ACC_T:(b + 1) * ACC_T], tb)
    tl = tb - Pt
    lo = (b * ACC_T + t) * C
    n = max(0, min(C, V - lo))
    acc, pick, lastpos, g3 = 0.0, -1, -1, np.inf
    for i in range(lo, lo + n):
        if w[i] > 0:
            lastpos = i
        acc += w[i]
        g3 = min(g3, abs(acc - tl))
        if acc > tl:
            pick = i
            break
    if pick < 0:
        pick = lastpos if lastpos >= 0 else lo
    return int(pick), min(g1, g2, g3) / scale


def accept_tree(p_logits, q_logits, tree, u, temperature, max_depth):
    """Mirror of the GPU acceptance walk.  tree: dict(token, trial_start, n_trials, trials) lists (the trials of a
    node are its children in draft-branch order, repeats included).  Each trial x is accepted when u < r(x) / q(x),
    r the current residual: p before any rejection, then max(p - c_j q, 0) / S_j after j rejections, c_1 = 1,
    c_{j+1} = c_j + S_j, S_j the sum of the numerator (equal to renormalising max(r - q, 0) after every rejection).
    Float64 with the kernel's single roundings and chunk_sums3 order; p and q from walk_probs, a bonus draw over
    block_weights' e * f.  Returns (accepted node ids, final token, uniforms used, bonus flag, smallest decision margin)."""
    cur, ui, path = 0, 0, []
    margin = np.inf
    take = lambda i: u[i] if i < len(u) else 0.5
    while True:
        nt = tree['n_trials'][cur]
        if nt == 0 or len(path) >= max_depth:
            e, f, bp, _ = block_weights(p_logits[cur], temperature)
            tok, mg = draw3(e * f, take(ui), bp)
            return path, tok, ui + 1, True, min(margin, mg)
        pp = walk_probs(p_logits[cur], temperature)
        qq = walk_probs(q_logits[cur], temperature)
        c, S, J, accepted, w = 0.0, 0.0, 0, -1, None
        t0 = tree['trial_start'][cur]
        for j in range(t0, t0 + nt):
            child = tree['trials'][j]
            x = tree['token'][child]
            px = pp[x]
            qx = qq[x]
            if J > 0:
                dx = px - c * qx
                px = dx / S if dx > 0.0 else 0.0
            uu = take(ui)
            ui += 1
            with np.errstate(divide='ignore', invalid='ignore'):
                ratio = np.float64(px) / np.float64(qx)
            margin = min(margin, abs(uu - ratio))
            if uu < ratio:
                accepted = child
                break
            c = 1.0 if J == 0 else c + S
            J += 1
            d = pp - c * qq
            w = np.where(d > 0.0, d, 0.0)
            S = chunk_sums3(w)[2]
        if accepted >= 0:
            path.append(accepted)
            cur = accepted
            continue
        tok, mg = draw3(w, take(ui))
        return path, tok, ui + 1, False, min(margin, mg)


# ------------------------------------------------------------------------------------------- exact output law
def _one_level_law(p, q, children_tokens):
    """Output law of the acceptance rule at one node, given the drafted children (i.i.d. from q, in draw order)."""
    cur = p.copy()
    out = np.zeros_like(p)
    remaining = 1.0
    for x in children_tokens:
        a = min(1.0, cur[x] / q[x]) if q[x] > 0 else 1.0
        out[x] += remaining * a
        remaining *= (1.0 - a)
        d = np.maximum(cur - q, 0.0)
        if d.sum() > 0:
            cur = d / d.sum()
    return out + remaining * cur


def exact_first_token_distribution(p, q, n_branches, grouped=False):
    """Marginal law of the first emitted token when `n_branches` drafts are drawn i.i.d. from q and verified with
    the multi-branch rule, one trial per draft in draw order (duplicate tokens share a tree node but keep their
    trial slots).  `grouped=True` tries duplicates back to back instead (first-draw order of distinct tokens), the
    ordering the rule must not use.  Enumerates all V^n draft outcomes."""
    V = len(p)
    law = np.zeros(V)
    for drafts in product(range(V), repeat=n_branches):
        prob = float(np.prod([q[d] for d in drafts]))
        if prob == 0.0:
            continue
        tried = list(drafts)
        if grouped:
            order = list(dict.fromkeys(drafts))
            tried = [x for x in order for d in drafts if d == x]
        law += prob * _one_level_law(p, q, tried)
    return law
