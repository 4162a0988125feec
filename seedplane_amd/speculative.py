"""Speculative decoding on MI355X.

Reference API (seedplane/speculative.py:1-111), same names, decisions and exceptions:
  ForestNode, SpeculativeForest.build / .paths / .roots / .node_count, Verification, verify_greedy(committed,
  forest, target_logits), CommitLedger(tokens, commits).frontier / .commit().
Additions (the reference prototype calls the target one position at a time and has no batched tree verifier):
  * flatten(): the forest as node arrays (node 0 = root = last committed token), children contiguous, with the
    number of branches that drew each node (`mult`).
  * verify_greedy_ids(): verify_greedy's decision procedure over target argmax ids instead of logits rows.
  * TreeVerifier: one tree-masked target pass over every node (HIP engine), greedy verification identical to
    verify_greedy, stochastic acceptance with residual resampling (GPU kernel), and KV compaction of the accepted
    path.
  * TreeDrafter: a drafter engine proposing `branches x depth` tokens by seeded sampling from its own distribution.
  * uniforms(): the seeded counter-based uniform stream (SplitMix64).
"""
import ctypes
from dataclasses import dataclass, field
from typing import Callable, Iterable, Sequence

import numpy as np

MASK64 = (1 << 64) - 1


# ===================================================================================== reference API
@dataclass
class ForestNode:
    token: int
    children: dict = field(default_factory=dict)


@dataclass
class SpeculativeForest:
    roots: dict = field(default_factory=dict)
    paths: list = field(default_factory=list)

    @classmethod
    def build(cls, branches: Iterable[Iterable[int]]) -> 'SpeculativeForest':
        """Trie of draft branches; empty branches are skipped, duplicates kept in `paths` (speculative.py:24-37)."""
        forest = cls()
        for branch in branches:
            path = tuple(int(token) for token in branch)
            if not path:
                continue
            forest.paths.append(path)
            children = forest.roots
            for token in path:
                node = children.get(token)
                if node is None:
                    node = children[token] = ForestNode(token)
                children = node.children
        return forest

    @property
    def node_count(self) -> int:
        def count(children):
            return sum(1 + count(node.children) for node in children.values())
        return count(self.roots)


@dataclass(frozen=True)
class Verification:
    emitted: tuple
    accepted_draft_tokens: int
    rejected: bool
    target_steps: int
    branch: tuple


def _first_max(values) -> int:
    best = 0
    for i in range(1, len(values)):
        if values[i] > values[best]:
            best = i
    return best


def verify_greedy_ids(committed: Sequence[int], forest: SpeculativeForest,
                      target_argmax: Callable[[tuple], int]) -> Verification:
    """verify_greedy with `target_argmax(prefix)` returning the target's greedy id directly."""
    base = tuple(int(t) for t in committed)
    if not forest.paths:
        return Verification((int(target_argmax(base)),), 0, False, 1, ())
    best = None
    for path in forest.paths:
        accepted = []
        steps = 0
        rejected = False
        for draft_token in path:
            target_token = int(target_argmax(base + tuple(accepted)))
            steps += 1
            if draft_token != target_token:
                accepted.append(target_token)
                rejected = True
                break
            accepted.append(draft_token)
        result = Verification(tuple(accepted), len(accepted) - int(rejected), rejected, steps, path)
        rank = (result.accepted_draft_tokens, len(result.emitted))
        if best is None or rank > (best.accepted_draft_tokens, len(best.emitted)):
            best = result
    return best


def verify_greedy(committed: Sequence[int], forest: SpeculativeForest,
                  target_logits: Callable[[tuple], Sequence[float]]) -> Verification:
    """Verify every draft path, then choose the longest exact greedy continuation (speculative.py:55-92).

    `target_logits(prefix)` returns target-model logits for the next token; the first disagreement emits the
    target token as correction; an empty forest falls back to one target token; ties keep branch input order."""
    def argmax(prefix):
        logits = target_logits(prefix)
        if not len(logits):
            raise ValueError('target returned empty logits')
        return _first_max(logits)
    return verify_greedy_ids(committed, forest, argmax)


@dataclass
class CommitLedger:
    """Committed token frontier; speculative state never mutates it pre-commit (speculative.py:95-111)."""
    tokens: list = field(default_factory=list)
    commits: int = 0

    @property
    def frontier(self) -> int:
        return len(self.tokens)

    def commit(self, verification: Verification) -> tuple:
        if not verification.emitted:
            raise ValueError('cannot commit an empty verification')
        committed = verification.emitted
        self.tokens.extend(committed)
        self.commits += 1
        return committed


# ===================================================================================== tree layout
@dataclass
class FlatTree:
    """Node arrays of a draft tree; node 0 is the root (the last committed token)."""
    token: list
    parent: list
    depth: list
    first_child: list
    n_children: list
    mult: list
    trial_start: list
    n_trials: list
    trials: list

    @property
    def size(self):
        return len(self.token)

    @property
    def max_depth(self):
        return max(self.depth)

    def ancestors_mask(self, i):
        m = 0
        while i >= 0:
            m |= 1 << i
            i = self.parent[i]
        return m

    def column_arrays(self):
        """(token int32, depth int32, ancestor masks uint64) arrays, computed once per tree."""
        cached = getattr(self, '_cols', None)
        if cached is None:
            masks = [0] * self.size
            for i in range(self.size):                     # parents precede children: one pass
                p = self.parent[i]
                masks[i] = (1 << i) | (masks[p] if p >= 0 else 0)
            cached = self._cols = (np.asarray(self.token, dtype=np.int32), np.asarray(self.depth, dtype=np.int32),
                                   np.asarray(masks, dtype=np.uint64))
        return cached

    def child(self, node, token):
        c0 = self.first_child[node]
        for c in range(c0, c0 + self.n_children[node]):
            if self.token[c] == token:
                return c
        return -1

    def node_of_prefix(self, prefix):
        """Node reached by following `prefix` (draft tokens after the root), or -1."""
        n = 0
        for t in prefix:
            n = self.child(n, t)
            if n < 0:
                return -1
        return n


def flatten(root_token: int, branches: Iterable[Iterable[int]]) -> FlatTree:
    """Breadth-first node arrays: children of a node contiguous, in first-draw order; mult = branches through the
    node.  The acceptance trials of a node are its children in draft-branch order, one per branch that continues
    through the node (repeats kept in place): the branches' draws there are i.i.d. from the drafter, and trying them
    in draw order is what keeps the multi-branch rule exact (grouping repeats back to back does not)."""
    paths = [tuple(int(t) for t in b) for b in branches]
    paths = [p for p in paths if p]
    token, parent, depth, mult = [int(root_token)], [-1], [0], [len(paths)]
    first_child, n_children = [-1], [0]
    node_trials = {}
    level = [(0, paths)]            # (node, branches passing through it, in input order)
    while level:
        nxt = []
        for node, bs in level:
            groups, order = {}, []
            seq = []
            for b in bs:
                d = depth[node]
                if len(b) <= d:
                    continue
                t = b[d]
                if t not in groups:
                    groups[t] = []
                    order.append(t)
                groups[t].append(b)
                seq.append(t)
            if order:
                first_child[node] = len(token)
                n_children[node] = len(order)
            index_of = {}
            for t in order:
                idx = len(token)
                index_of[t] = idx
                token.append(t); parent.append(node); depth.append(depth[node] + 1)
                mult.append(len(groups[t])); first_child.append(-1); n_children.append(0)
                nxt.append((idx, groups[t]))
            node_trials[node] = [index_of[t] for t in seq]
        level = nxt
    trial_start, n_trials, trials = [], [], []
    for i in range(len(token)):
        ts = node_trials.get(i, [])
        trial_start.append(len(trials)); n_trials.append(len(ts)); trials.extend(ts)
    return FlatTree(token, parent, depth, first_child, n_children, mult, trial_start, n_trials, trials)


# ===================================================================================== seeded uniforms
def _splitmix64(x):
    x = (x + 0x9E3779B97F4A7C15) & MASK64
    z = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def _splitmix64_np(x):
    """_splitmix64 on a uint64 array (numpy integer arithmetic wraps modulo 2^64)."""
    x = x + np.uint64(0x9E3779B97F4A7C15)
    z = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def uniforms(seed, step, n):
    """Counter-based uniforms in [0, 1): u_i = (splitmix64(splitmix64(seed) ^ (step * 2^20 + i)) >> 11) * 2^-53.
    (The top 53 bits convert to float64 exactly, so the values do not depend on how the integers are computed.)"""
    s = np.uint64(_splitmix64(int(seed) & MASK64))
    ctr = (np.uint64((int(step) << 20) & MASK64) + np.arange(n, dtype=np.uint64))
    return (_splitmix64_np(s ^ ctr) >> np.uint64(11)).astype(np.float64) * 2.0 ** -53


# ===================================================================================== GPU verification
class TreeVerifier:
    """Tree-masked verification on a Qwen2Engine (HIP).  The cache holds every committed token but the last, which
    is passed as the root; after `commit`, the cache holds everything emitted except the new last token."""

    def __init__(self, engine):
        import torch
        from . import _lib
        self.engine = engine
        self._lib = _lib
        self.torch = torch
        self._out = {}
        self._colbuf = np.empty(64, dtype=_lib.TOKEN_DTYPE)       # the columns of the latest pass (forward)
        self._colbuf_ptr = self._colbuf.ctypes.data

    def forward(self, cache, tree: FlatTree, logits_out=None, graph=False, ids=True):
        """One pass over every node: node i is written at cache position cache.length + i, RoPE position
        cache.length + depth[i], and attends to the cache before the root plus its own ancestors.  Returns the
        greedy ids per node; logits [nodes, vocab] go to `logits_out` when given.  With ids=False (acceptance
        sampling needs the logits only) no argmax runs and the call does not wait for the GPU: it returns the logits,
        in `logits_out` or, without it, as a view of the engine's own logits buffer (no copy; valid until the
        engine's next forward call)."""
        e = self.engine
        n = tree.size
        self._fill_columns(cache, tree, self._colbuf_ptr)
        flags = self._lib.SP_F_LOGITS | (self._lib.SP_F_GRAPH if graph else 0)
        out = e.run_raw(n, self._colbuf_ptr, flags, logits_out=logits_out, want_ids=ids)
        if ids:
            return out
        return logits_out if logits_out is not None else e.logits_view(n)

    def columns(self, cache, tree: FlatTree):
        """The engine columns of one tree pass (a numpy array of _lib.TOKEN_DTYPE): node i in slot
        (cache.length + i) mod slots, which is tree slot i of the pass, at RoPE position cache.length + depth[i],
        seeing the cached positions before the root (the window's part of them) and the tree nodes of its mask."""
        cols = np.empty(tree.size, dtype=self._lib.TOKEN_DTYPE)
        self._fill_columns(cache, tree, cols.ctypes.data)
        return cols

    def _fill_columns(self, cache, tree: FlatTree, dst):
        """columns() into the TOKEN_DTYPE records at address dst (room for tree.size records)."""
        e = self.engine
        e._check_cache(cache)
        n = tree.size
        if n > min(e.max_tokens, 64):
            raise ValueError(f'tree of {n} nodes exceeds the engine max_tokens / 64-node mask')
        P = cache.length
        if cache.window is None and P + n > cache.capacity:
            raise ValueError(f'KV cache capacity {cache.capacity} exceeded')
        ptrs = getattr(tree, '_col_ptrs', None)
        if ptrs is None:                               # addresses of the tree's arrays (they live with the tree)
            ptrs = tree._col_ptrs = tuple(a.ctypes.data for a in tree.column_arrays())
        self._lib.check(e.lib.sp_tree_columns(n, *ptrs, cache.seq, P, e._pool_slots, cache.window or 0, dst))

    def commit(self, cache, tree: FlatTree, path_nodes):
        """Keep the root and the accepted path nodes (in order) in the cache: their K/V move to consecutive slots
        after the root, and cache.length = root position + 1 + len(path_nodes)."""
        e = self.engine
        P, S = cache.length, e._pool_slots
        src = [(P + node) % S for node in path_nodes]
        dst = [(P + 1 + i) % S for i in range(len(path_nodes))]
        moves = [(s, d) for s, d in zip(src, dst) if s != d]
        if moves:
            a = np.array([m[0] for m in moves], dtype=np.int32)
            b = np.array([m[1] for m in moves], dtype=np.int32)
            self._lib.check(e.lib.sp_engine_kv_move(e.h, cache.seq, len(moves), ctypes.c_void_p(a.ctypes.data),
                                                    ctypes.c_void_p(b.ctypes.data)), e.h)
        cache.length = P + 1 + len(path_nodes)

    def verify_greedy(self, cache, committed, forest: SpeculativeForest):
        """verify_greedy over one tree pass; the decision is identical to the reference's verify_greedy fed with
        this engine's logits.  Commits the kept tokens (all emitted but the last) to the cache."""
        root = int(committed[-1])
        tree = flatten(root, forest.paths)
        ids = self.forward(cache, tree)

        def argmax(prefix):
            node = tree.node_of_prefix(prefix[len(committed):])
            return int(ids[node])
        v = verify_greedy_ids(committed, forest, argmax)
        kept = []
        node = 0
        for t in v.emitted[:-1]:
            node = tree.child(node, t)
            kept.append(node)
        self.commit(cache, tree, kept)
        return v

    def accept(self, p_logits, q_logits, tree: FlatTree, u, temperature, q_index=None):
        """GPU acceptance walk (sp_op_accept_tree_host: the tree arrays and uniforms go from host memory straight to
        the kernel, no copy on the stream).  p_logits: device tensor [nodes, vocab]; q_logits: [nodes, vocab], or any
        [rows, vocab] with `q_index` giving node i's row (sp_op_accept_tree_rows; TreeDrafter.q_index).
        Returns (accepted node ids, final token, uniforms used, bonus)."""
        torch = self.torch
        dev = p_logits.device
        V = p_logits.shape[1]
        md = max(1, tree.max_depth)
        # the int32 tree arrays, concatenated once per tree
        acc = getattr(tree, '_acc', None)
        if acc is None:
            ints = [tree.token, tree.trial_start, tree.n_trials, tree.trials if len(tree.trials) else [0]]
            sizes = [len(x) for x in ints]
            acc = tree._acc = (np.concatenate([np.asarray(x, dtype=np.int32) for x in ints]),
                               [int(o) for o in np.cumsum([0] + sizes[:-1])])
        flat, rel = acc
        uu = np.ascontiguousarray(u, dtype=np.float64)
        out = self._out.get((dev, md))
        if out is None:
            out = self._out[(dev, md)] = torch.empty(md + 4, dtype=torch.int32, device=dev)
        res = np.empty(md + 4, dtype=np.int32)
        base = flat.ctypes.data
        at = lambda o: ctypes.c_void_p(base + 4 * o)
        ptr = lambda t: ctypes.c_void_p(t.data_ptr())
        stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        if q_logits.stride(0) != p_logits.stride(0):
            raise ValueError('p and q logits rows must have the same stride')
        if q_index is None:
            self._lib.check(self.engine.lib.sp_op_accept_tree_host(
                ptr(p_logits), ptr(q_logits), V, p_logits.stride(0), tree.size, at(rel[0]), at(rel[1]), at(rel[2]),
                at(rel[3]), len(tree.trials), ctypes.c_void_p(uu.ctypes.data), len(uu), float(temperature), md,
                ptr(out), stream, res.ctypes.data_as(ctypes.c_void_p)))
        else:
            qi = np.ascontiguousarray(q_index, dtype=np.int32)
            if len(qi) != tree.size:
                raise ValueError('q_index needs one row per tree node')
            self._lib.check(self.engine.lib.sp_op_accept_tree_rows(
                ptr(p_logits), ptr(q_logits), q_logits.shape[0], V, p_logits.stride(0), tree.size, at(rel[0]),
                at(rel[1]), at(rel[2]), at(rel[3]), len(tree.trials), ctypes.c_void_p(qi.ctypes.data),
                ctypes.c_void_p(uu.ctypes.data), len(uu), float(temperature), md, ptr(out), stream,
                res.ctypes.data_as(ctypes.c_void_p)))
        o = res.tolist()
        k = o[0]
        return o[1:1 + k], o[md + 1], o[md + 2], bool(o[md + 3])

def sample_rows(lib_engine, logits, rows, u, temperature):
    """Seeded inverse-CDF draws from softmax(logits[rows[s]] / T) on the GPU (sp_op_sample)."""
    import torch
    from . import _lib
    dev = logits.device
    r = torch.tensor(list(rows), dtype=torch.int32, device=dev)
    ud = torch.tensor(np.asarray(u, dtype=np.float64), device=dev)
    out = torch.empty(len(rows), dtype=torch.int32, device=dev)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    _lib.check(lib_engine.sp_op_sample(ptr(logits), logits.shape[1], logits.stride(0), ptr(r), ptr(ud), len(rows),
                                       float(temperature), ptr(out), stream))
    return out.cpu().tolist()


class TreeDrafter:
    """Proposes `branches` draft continuations of `depth` tokens by seeded sampling from a drafter engine, with every
    level on the device.

    The drafter's cache holds the committed tokens it has processed; `propose` first runs the pending committed
    tokens (ending with the root) and draws every branch's first token from the root's row.  Level l = 1 .. depth-1
    then runs one column per branch: branch b's level-l token as drafted node (l - 1) * B + b, in the slots after the
    root, seeing the committed range and, through its tree mask, the canonical node of its branch at every earlier
    level and itself.  A branch's canonical node is the first branch with the same prefix (sp_op_draft_link), and
    every branch draws its next token from its canonical column's row, so the branches through one tree node draw
    independently from that node's one distribution (what the multi-branch acceptance rule assumes).  Tokens,
    canonical indices and masks stay on the device (the columns read them through SP_F_DEVCOLS); the host reads the
    drafted tokens and canonical indices once, after the last level."""

    def __init__(self, engine):
        self.engine = engine
        self._bufs = {}
        self._node_of, self._index, self._L = {}, {}, -1
        self.q_rows = None

    def _buffers(self, B, depth):
        b = self._bufs.get((B, depth))
        if b is None:
            import torch
            e = self.engine
            i32 = dict(dtype=torch.int32, device=e.device)
            b = self._bufs[(B, depth)] = dict(
                q=torch.empty((1 + B * (depth - 1), e.vocab), dtype=torch.float32, device=e.device),
                toks=torch.zeros((depth, B), **i32), canon=torch.zeros((depth, B), **i32),
                masks=torch.zeros(B, dtype=torch.int64, device=e.device), rows=torch.zeros(B, **i32),
                zero=torch.zeros(B, **i32), u=torch.zeros(B * depth, dtype=torch.float64, device=e.device),
                u_host=torch.zeros(B * depth, dtype=torch.float64).pin_memory())
        return b

    def propose(self, cache, pending, n_branches, depth, temperature, u, graph=False):
        """Returns (branches, rows, used): `rows` maps a drafted prefix (tuple of tokens after the root, shorter than
        `depth`) to the drafter logits row there, a view of `self.q_rows` (overwritten by the next proposal);
        `q_index(tree)` gives the same rows by index; `used` = uniforms consumed (one per branch per level)."""
        import torch
        from . import _lib
        e = self.engine
        B = n_branches
        if B < 1 or depth < 1 or B * max(depth - 1, 1) > 64:
            raise ValueError('n_branches x (depth - 1) drafted nodes must be in [1, 64]')
        if len(u) < B * depth:
            raise ValueError('need n_branches x depth uniforms')
        bf = self._buffers(B, depth)
        q, toks, canon, masks, rows = bf['q'], bf['toks'], bf['canon'], bf['masks'], bf['rows']
        L = cache.length + len(pending) - 1          # position of the root
        if cache.window is None and L + 1 + B * (depth - 1) > cache.capacity:
            raise ValueError('drafter cache too small for the draft tree')
        # the uniforms go up from pinned memory without waiting (the last proposal's copy ended at its read-back)
        bf['u_host'].numpy()[:] = np.asarray(u[:B * depth], dtype=np.float64)
        ud = bf['u']
        ud.copy_(bf['u_host'], non_blocking=True)
        logits, cache = e.forward(pending, cache)
        q[0].copy_(logits[0])
        lib, V, S = e.lib, e.vocab, e._pool_slots
        ptr = lambda t: ctypes.c_void_p(t.data_ptr())
        stream = ctypes.c_void_p(torch.cuda.current_stream(e.device).cuda_stream)
        T = float(temperature)
        _lib.check(lib.sp_op_sample(ptr(q), V, V, ptr(bf['zero']), ptr(ud), B, T, ptr(toks[0]), stream))
        base = (L + 1) % S
        try:
            for lv in range(depth - 1):
                _lib.check(lib.sp_op_draft_link(ptr(toks), B, lv, ptr(canon), ptr(masks), ptr(rows), stream))
                pos = L + 1 + lv
                lo = 0 if cache.window is None else max(0, pos - cache.window + 1)
                cols = [(0, cache.seq, pos, (L + 1 + lv * B + b) % S, lo, L, base, B * (lv + 1), 0) for b in range(B)]
                _lib.check(lib.sp_engine_set_device_columns(e.h, ptr(toks[lv]), ptr(masks)), e.h)
                out = q[1 + lv * B:1 + (lv + 1) * B]
                e.run(cols, _lib.SP_F_LOGITS | _lib.SP_F_DEVCOLS, logits_out=out)
                _lib.check(lib.sp_op_sample(ptr(out), V, V, ptr(rows), ptr(ud[B * (lv + 1):]), B, T,
                                            ptr(toks[lv + 1]), stream))
        finally:
            _lib.check(lib.sp_engine_set_device_columns(e.h, None, None), e.h)
        host = torch.cat([toks.flatten(), canon.flatten()]).cpu().numpy()   # the proposal's one read-back
        tk, cn = host[:depth * B].reshape(depth, B), host[depth * B:].reshape(depth, B)
        branches = [[int(tk[lv, b]) for lv in range(depth)] for b in range(B)]
        self._node_of, self._index = {}, {(): 0}
        out_rows = {(): q[0]}
        for lv in range(depth - 1):
            for b in range(B):
                pref = tuple(branches[b][:lv + 1])
                j = lv * B + int(cn[lv, b])          # the same for every branch with this prefix
                self._node_of[pref] = j
                self._index[pref] = 1 + j
                out_rows[pref] = q[1 + j]
        self._L = L
        self.q_rows = q
        return branches, out_rows, B * depth

    def q_index(self, tree: FlatTree):
        """Row of `self.q_rows` holding the drafter's distribution at each node of `tree` (the flattened last
        proposal); leaves (never read by the acceptance walk) get row 0."""
        out, prefixes = [0] * tree.size, [()]
        for i in range(1, tree.size):
            prefixes.append(prefixes[tree.parent[i]] + (tree.token[i],))
        for i, pref in enumerate(prefixes):
            if tree.n_children[i]:
                out[i] = self._index[pref]
        return out

    def commit(self, cache, accepted_tokens):
        """Keep the drafted nodes on the accepted path (those the drafter processed) after the root."""
        kept, pref = [], ()
        for t in accepted_tokens:
            pref = pref + (t,)
            j = self._node_of.get(pref)
            if j is None:
                break
            kept.append(j)
        # drafted node j lives at slot L + 1 + j; the root itself is at L
        e = self.engine
        S = e._pool_slots
        moves = [((self._L + 1 + j) % S, (self._L + 1 + i) % S) for i, j in enumerate(kept) if j != i]
        if moves:
            a = np.array([m[0] for m in moves], dtype=np.int32)
            b = np.array([m[1] for m in moves], dtype=np.int32)
            from . import _lib
            _lib.check(e.lib.sp_engine_kv_move(e.h, cache.seq, len(moves), ctypes.c_void_p(a.ctypes.data),
                                               ctypes.c_void_p(b.ctypes.data)), e.h)
        cache.length = self._L + 1 + len(kept)
        return len(kept)


def q_rows_for_tree(tree: FlatTree, rows, vocab, device):
    """Drafter logits aligned with the target tree's node order (rows of leaves are zero; they are never read)."""
    import torch
    q = torch.zeros((tree.size, vocab), dtype=torch.float32, device=device)
    prefixes = [()]
    for i in range(1, tree.size):
        prefixes.append(prefixes[tree.parent[i]] + (tree.token[i],))
    for i, pref in enumerate(prefixes):
        if tree.n_children[i] and pref in rows:
            q[i].copy_(rows[pref])
    return q


@dataclass
class SpecStats:
    steps: int = 0
    emitted: int = 0
    accepted: int = 0
    bonus: int = 0
    nodes: int = 0


class SpeculativeLoop:
    """Tree speculative sampling, one step at a time: each step the drafter proposes n_branches x depth tokens, the
    target verifies all nodes in one pass, the acceptance kernel keeps a prefix of one branch plus one corrected or
    bonus token.  The constructor prefills both caches with the prompt (all but its last token, the first step's
    root), so `step()` does only a step's work.  `capacity`: cache positions (default: the prompt + 4096)."""

    def __init__(self, target, drafter, prompt, n_branches=8, depth=4, temperature=0.8, seed=0, window=None,
                 capacity=None, stats=None):
        if len(prompt) < 1:
            raise ValueError('prompt cannot be empty')
        cap = capacity if capacity is not None else len(prompt) + 4096
        self.target, self.drafter = target, drafter
        self.n_branches, self.depth, self.temperature, self.seed = n_branches, depth, temperature, seed
        self.tcache = target.new_cache(cap, window=window)
        self.dcache = drafter.engine.new_cache(cap, window=window)
        self.verifier = TreeVerifier(target)
        self.committed = [int(t) for t in prompt]
        self.stats = stats if stats is not None else SpecStats()
        self._step = 0
        if len(self.committed) > 1:
            target.forward(self.committed[:-1], self.tcache)
            drafter.engine.forward(self.committed[:-1], self.dcache)

    def step(self):
        """One speculative step; returns the emitted tokens (accepted drafts + the corrected or bonus token)."""
        B, depth, T = self.n_branches, self.depth, self.temperature
        u = uniforms(self.seed, self._step, B * depth + 64)
        self._step += 1
        pending = self.committed[self.dcache.length:]
        branches, rows, used = self.drafter.propose(self.dcache, pending, B, depth, T, u)
        tree = flatten(self.committed[-1], branches)
        p = self.verifier.forward(self.tcache, tree, ids=False)    # the target engine's own logits rows, no copy
        path, final, _, bonus = self.verifier.accept(p, self.drafter.q_rows, tree, u[used:], T,
                                                     q_index=self.drafter.q_index(tree))
        acc_tokens = [tree.token[n] for n in path]
        self.verifier.commit(self.tcache, tree, path)
        self.drafter.commit(self.dcache, acc_tokens)
        emitted = acc_tokens + [int(final)]
        self.committed += emitted
        st = self.stats
        st.steps += 1; st.emitted += len(emitted); st.accepted += len(path); st.bonus += int(bonus)
        st.nodes += tree.size - 1
        return emitted


def speculative_generate(target, drafter, prompt, steps, n_branches=8, depth=4, temperature=0.8, seed=0,
                         window=None, stats=None):
    """`steps` steps of SpeculativeLoop over a fresh pair of caches.  Returns the generated tokens (after the
    prompt)."""
    loop = SpeculativeLoop(target, drafter, prompt, n_branches, depth, temperature, seed, window,
                           capacity=len(prompt) + steps * (depth + 1) + 2 * 64, stats=stats)
    out = []
    for _ in range(steps):
        out += loop.step()
    return out
