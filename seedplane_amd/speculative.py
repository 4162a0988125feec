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

    def accept(self, p_logits, q_logits, tree: FlatTree, u, temperature):
        """GPU acceptance walk (sp_op_accept_tree_host: the tree arrays and uniforms go from host memory straight to
        the kernel, no copy on the stream).  p_logits / q_logits: device tensors [nodes, vocab].
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
        self._lib.check(self.engine.lib.sp_op_accept_tree_host(
            ptr(p_logits), ptr(q_logits), V, p_logits.stride(0), tree.size, at(rel[0]), at(rel[1]), at(rel[2]),
            at(rel[3]), len(tree.trials), ctypes.c_void_p(uu.ctypes.data), len(uu), float(temperature), md, ptr(out),
            stream, res.ctypes.data_as(ctypes.c_void_p)))
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
    """Proposes `branches` draft continuations of `depth` tokens by seeded sampling from a drafter engine.

    The drafter's cache holds the committed tokens it has processed; `propose` first runs the pending committed
    tokens (ending with the root), samples every branch's first token from the root distribution, then runs one
    tree-masked pass per level over the new nodes and samples each branch's next token from its node's distribution.
    Branches sharing a node draw independently from the same distribution (what the multi-branch acceptance rule
    assumes)."""

    def __init__(self, engine):
        self.engine = engine
        self.verifier = TreeVerifier(engine)
        self._tok, self._par, self._lvl = [], [], []

    def _mask(self, j):
        m = 0
        while j >= 0:
            m |= 1 << j
            j = self._par[j]
        return m

    def propose(self, cache, pending, n_branches, depth, temperature, u, graph=False):
        """Returns (branches, rows, used): `rows` maps a drafted prefix (tuple of tokens after the root) to the
        drafter logits row (device tensor) there; `used` = uniforms consumed (one per branch per level)."""
        import torch
        from . import _lib
        e = self.engine
        logits, cache = e.forward(pending, cache)
        L = cache.length - 1                         # position of the root
        rows = {(): logits[0]}
        ui = 0
        first = sample_rows(e.lib, logits, [0] * n_branches, u[ui:ui + n_branches], temperature)
        ui += n_branches
        branches = [[t] for t in first]
        self._tok, self._par, self._lvl = [], [], []
        node_of = {}                                 # prefix -> drafter node index
        S = e._pool_slots
        V = e.vocab
        for level in range(1, depth):
            new_nodes = []
            for b in branches:
                pref = tuple(b)
                if pref not in node_of:
                    node_of[pref] = len(self._tok)
                    self._tok.append(pref[-1])
                    self._par.append(node_of.get(pref[:-1], -1))
                    self._lvl.append(level)
                    new_nodes.append(node_of[pref])
            n_tree = len(self._tok)
            if L + 1 + n_tree > cache.capacity and cache.window is None:
                raise ValueError('drafter cache too small for the draft tree')
            cols = []
            for j in new_nodes:
                pos = L + self._lvl[j]
                lo = 0 if cache.window is None else max(0, pos - cache.window + 1)
                cols.append((self._tok[j], cache.seq, pos, (L + 1 + j) % S, lo, L, (L + 1) % S, n_tree, self._mask(j)))
            out = torch.empty((len(cols), V), dtype=torch.float32, device=e.device)
            e.run(cols, _lib.SP_F_LOGITS, logits_out=out)
            for r, j in enumerate(new_nodes):
                pref = next(p for p, n in node_of.items() if n == j)
                rows[pref] = out[r]
            row_of_branch = [new_nodes.index(node_of[tuple(b)]) for b in branches]
            nxt = sample_rows(e.lib, out, row_of_branch, u[ui:ui + n_branches], temperature)
            ui += n_branches
            for b, t in zip(branches, nxt):
                b.append(t)
        self._node_of = node_of
        self._L = L
        return branches, rows, ui

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


def speculative_generate(target, drafter, prompt, steps, n_branches=8, depth=4, temperature=0.8, seed=0,
                         window=None, stats=None):
    """Tree speculative sampling: each step the drafter proposes n_branches x depth tokens, the target verifies all
    nodes in one pass, the acceptance kernel keeps a prefix of one branch plus one corrected or bonus token.
    Returns the generated tokens (after the prompt)."""
    import torch
    if len(prompt) < 1:
        raise ValueError('prompt cannot be empty')
    cap = len(prompt) + steps * (depth + 1) + 2 * 64
    tcache = target.new_cache(cap, window=window)
    dcache = drafter.engine.new_cache(cap, window=window)
    verifier = TreeVerifier(target)
    committed = [int(t) for t in prompt]
    if len(committed) > 1:
        target.forward(committed[:-1], tcache)
    out = []
    st = stats if stats is not None else SpecStats()
    for step in range(steps):
        u = uniforms(seed, step, n_branches * depth + 64)
        pending = committed[dcache.length:]
        branches, rows, used = drafter.propose(dcache, pending, n_branches, depth, temperature, u)
        tree = flatten(committed[-1], branches)
        p = verifier.forward(tcache, tree, ids=False)          # the target engine's own logits rows, no copy
        q = q_rows_for_tree(tree, rows, target.vocab, target.device)
        path, final, _, bonus = verifier.accept(p, q, tree, u[used:], temperature)
        acc_tokens = [tree.token[n] for n in path]
        verifier.commit(tcache, tree, path)
        drafter.commit(dcache, acc_tokens)
        emitted = acc_tokens + [int(final)]
        committed += emitted
        out += emitted
        st.steps += 1; st.emitted += len(emitted); st.accepted += len(path); st.bonus += int(bonus)
        st.nodes += tree.size - 1
    return out
