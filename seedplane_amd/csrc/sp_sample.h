// Seeded sampling and speculative acceptance on the GPU, in float64.
//
// Every distribution is softmax(logits / T) over a full fp32 logits row, computed in fp64 with one fixed summation
// order so the CPU oracle can restate it: the row is cut into SMP_THREADS contiguous chunks of
// C = ceil(V / SMP_THREADS) entries; each chunk is summed sequentially in index order, and the chunk sums are added
// sequentially in chunk order.  Inverse-CDF draws use the same chunks: target = u * Z, the chunk whose prefix range
// holds the target is found from the sequential chunk prefixes, then scanned sequentially.
//
// Acceptance (speculative sampling with a residual, Leviathan et al. 2023 / Chen et al. 2023, extended to a tree
// of drafts as in SpecInfer, Miao et al. 2023): at a node, its trials -- the child each draft branch through the
// node drew, in branch (= draw) order, repeats kept in place -- are tried in turn; a child x is accepted iff
// u < p(x) / q(x) with p the target's current distribution and q the drafter's distribution at that node; each
// rejection replaces p by the residual norm(max(p - q, 0)).  If every child is rejected, the next token is drawn from the residual; if the
// accepted node has no children, a bonus token is drawn from the target's distribution there.  Uniforms are
// consumed in that order, one per trial and one for the final draw.
#pragma once
#include "sp_device.h"

constexpr int SMP_THREADS = 1024;      // chunks per row

// Seeded draws on many blocks per row, three launches, in the summation order stated at the top of this file:
//   k_smp_max   SMX_BLOCKS blocks per draw: partial maxima of the row (a maximum is exact in any order);
//   k_smp_sum   SMP_THREADS / SMS_CPB blocks per draw: the row maximum m from the partial maxima, then the sums of
//               SMS_CPB chunks: the block's threads compute the weights exp((l_i - m) / T) of a window of entries into
//               LDS, and one thread per chunk adds its chunk's entries of the window in index order, carrying the
//               chunk's running sum from window to window (the same additions as one thread summing its chunk);
//   k_smp_draw  one block per draw: thread 0 adds the chunk sums in chunk order (the total and the exclusive
//               prefixes), the chunk holding target = u * total is found, and its entries are scanned in index order
//               (weights computed by the block a window at a time, running sum by thread 0).
// Every total, prefix and comparison is that order's, so a sequential evaluation reproduces every draw bit for bit;
// the fallbacks: a chunk with no running sum above the target gives its last positive-weight index, no positive
// weight where the target fell gives the last positive-weight index of the row (0 if none).
// Scratch per draw: SMX_BLOCKS floats and SMP_THREADS doubles.
constexpr int SMX_BLOCKS = 64, SMS_CPB = 8, SMS_T = 256, SMS_WIN = 2048;

__device__ __forceinline__ double smp_weight(const float *l, int i, float m, double invT) {
    return exp(((double)l[i] - (double)m) * invT);
}

__device__ __forceinline__ float smp_row_max(const float *pmax) {
    float m = pmax[0];
    for (int j = 1; j < SMX_BLOCKS; ++j) m = fmaxf(m, pmax[j]);
    return m;
}

__global__ void __launch_bounds__(SMS_T) k_smp_max(const float *logits, int V, int ld, const int *rows, float *pmax) {
    __shared__ float red[SMS_T / 64];
    const int s = blockIdx.y, bk = blockIdx.x;
    const float *l = logits + (size_t)rows[s] * ld;
    const int per = (V + SMX_BLOCKS - 1) / SMX_BLOCKS;
    const int lo = bk * per, hi = min(V, lo + per);
    float m = -INFINITY;
    for (int i = lo + (int)threadIdx.x; i < hi; i += SMS_T) m = fmaxf(m, l[i]);
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = red[0];
        for (int j = 1; j < SMS_T / 64; ++j) t = fmaxf(t, red[j]);
        pmax[s * SMX_BLOCKS + bk] = t;
    }
}

__global__ void __launch_bounds__(SMS_T) k_smp_sum(const float *logits, int V, int ld, const int *rows, double invT,
                                                    const float *pmax, double *csum) {
    __shared__ double w[SMS_WIN];
    const int s = blockIdx.y;
    const float *l = logits + (size_t)rows[s] * ld;
    const float m = smp_row_max(pmax + s * SMX_BLOCKS);
    const int C = (V + SMP_THREADS - 1) / SMP_THREADS;
    const int c0 = blockIdx.x * SMS_CPB;
    const int lo = min(V, c0 * C), hi = min(V, (c0 + SMS_CPB) * C);
    const int t = threadIdx.x;
    // thread t < SMS_CPB owns chunk c0 + t: entries [clo, chi)
    const int clo = min(V, (c0 + t) * C), chi = min(V, (c0 + t + 1) * C);
    double acc = 0.0;
    for (int wlo = lo; wlo < hi; wlo += SMS_WIN) {
        const int whi = min(hi, wlo + SMS_WIN);
        for (int i = wlo + t; i < whi; i += SMS_T) w[i - wlo] = smp_weight(l, i, m, invT);
        __syncthreads();
        if (t < SMS_CPB) {
            const int a = max(clo, wlo), e = min(chi, whi);
            for (int i = a; i < e; ++i) acc += w[i - wlo];
        }
        __syncthreads();
    }
    if (t < SMS_CPB) csum[(size_t)s * SMP_THREADS + c0 + t] = acc;
}

__global__ void __launch_bounds__(SMS_T) k_smp_draw(const float *logits, int V, int ld, const int *rows,
                                                     const double *u, double invT, const float *pmax,
                                                     const double *csum, int *out) {
    __shared__ double pre[SMP_THREADS + 1];
    __shared__ double w[SMS_WIN + 16];
    __shared__ int sel, found;
    __shared__ int last[SMS_T / 64];
    const int s = blockIdx.x, t = threadIdx.x;
    const float *l = logits + (size_t)rows[s] * ld;
    const float m = smp_row_max(pmax + s * SMX_BLOCKS);
    const int C = (V + SMP_THREADS - 1) / SMP_THREADS;
    for (int j = t; j < SMP_THREADS; j += SMS_T) pre[j] = csum[(size_t)s * SMP_THREADS + j];
    if (t == 0) { sel = -1; found = -1; }
    __syncthreads();
    if (t == 0) {
        // the sums in chunk order; each batch of 32 is read into registers first, so the reads do not wait on the
        // prefixes written before them
        double p = 0.0;
        for (int j0 = 0; j0 < SMP_THREADS; j0 += 32) {
            double c[32];
#pragma unroll
            for (int k = 0; k < 32; ++k) c[k] = pre[j0 + k];
#pragma unroll
            for (int k = 0; k < 32; ++k) {
                pre[j0 + k] = p;
                p += c[k];
            }
        }
        pre[SMP_THREADS] = p;
    }
    __syncthreads();
    const double target = u[s] * pre[SMP_THREADS];
    for (int j = t; j < SMP_THREADS; j += SMS_T)
        if (target >= pre[j] && (j + 1 == SMP_THREADS || target < pre[j + 1])) sel = j;
    __syncthreads();
    if (sel >= 0) {
        // scan chunk sel from zero against target - prefix: the first index whose running sum exceeds it, else the
        // chunk's last positive-weight index
        const int clo = min(V, sel * C), chi = min(V, sel * C + C);
        const double tl = target - pre[sel];
        double acc = 0.0;
        int pick = -1, lastpos = -1;
        for (int wlo = clo; wlo < chi; wlo += SMS_WIN) {
            const int whi = min(chi, wlo + SMS_WIN);
            for (int i = wlo + t; i < whi; i += SMS_T) w[i - wlo] = smp_weight(l, i, m, invT);
            __syncthreads();
            if (t == 0 && pick < 0) {
                // in index order, 16 weights read ahead at a time (entries past the window read a zero pad and are
                // not visited)
                for (int i0 = wlo; i0 < whi && pick < 0; i0 += 16) {
                    double c[16];
#pragma unroll
                    for (int k = 0; k < 16; ++k) c[k] = w[i0 - wlo + k];
#pragma unroll
                    for (int k = 0; k < 16; ++k) {
                        const int i = i0 + k;
                        if (pick < 0 && i < whi) {
                            if (c[k] > 0.0) lastpos = i;
                            acc += c[k];
                            if (acc > tl) pick = i;
                        }
                    }
                }
                found = pick;
            }
            __syncthreads();
            if (found >= 0) break;
        }
        if (t == 0 && pick < 0) found = lastpos;
        __syncthreads();
    }
    if (found < 0) {
        // no positive weight where the target fell: the last positive-weight index of the row (0 if none)
        int best = 0;
        for (int i = t; i < V; i += SMS_T)
            if (smp_weight(l, i, m, invT) > 0.0) best = max(best, i);
        for (int o = 32; o > 0; o >>= 1) best = max(best, __shfl_xor(best, o, SP_WAVE));
        if ((t & 63) == 0) last[t >> 6] = best;
        __syncthreads();
        if (t == 0) {
            int b = last[0];
            for (int j = 1; j < SMS_T / 64; ++j) b = max(b, last[j]);
            found = b;
        }
        __syncthreads();
    }
    if (t == 0) out[s] = found;
}

// One level of a drafter's proposal on the device (one block, thread b = branch b < nb; tokens [levels][nb]): the
// branch's canonical branch at `level` -- the first branch whose tokens at levels 0..level equal its own, so every
// branch through a tree node draws from that node's one row -- then, for the level's columns, column b's tree mask
// (the canonical node of its branch at every earlier level, node index level' * nb + canonical, and the column
// itself) and the row its next token is drawn from (its canonical column).
__global__ void k_draft_link(const int *tokens, int nb, int level, int *canon, unsigned long long *masks, int *rows) {
    const int b = threadIdx.x;
    if (b >= nb) return;
    int c = b;
    for (int o = 0; o < b; ++o) {
        bool same = true;
        for (int lv = 0; lv <= level; ++lv) same = same && tokens[lv * nb + o] == tokens[lv * nb + b];
        if (same) { c = o; break; }
    }
    canon[level * nb + b] = c;
    unsigned long long m = 1ull << (level * nb + b);
    for (int lv = 0; lv < level; ++lv) m |= 1ull << (lv * nb + canon[lv * nb + b]);
    masks[b] = m;
    rows[b] = c;
}

// ---------------------------------------------------------------------------------------------------------------
// Tree acceptance on ACC_NB co-resident blocks (a plain launch: 64 blocks of 256 threads are all resident on the
// 256-CU chip once the stream's previous kernel has finished, and every exchange wait is bounded, so a block that
// never arrives ends the launch with an error instead of a hang; a cooperative launch enqueued behind a running
// kernel slowed that kernel by ~10 %).  The vocabulary is cut into ACC_NB x ACC_T contiguous chunks of
// C = ceil(V / (ACC_NB * ACC_T)) entries; thread t of block b owns chunk b * ACC_T + t and keeps its logits' weights
// in registers.  Sums are taken sequentially inside a chunk, then over the ACC_T chunk sums of a block (butterfly in
// each wave, wave sums in order: the block partial), then sequentially over the ACC_NB block partials.  Block partials are all-gathered through
// tagged 64-bit words (32-bit payload + 32-bit tag, single-copy atomic; relaxed agent-scope atomics, no fences), so
// every block holds every partial and takes every accept / reject decision itself.
//
// Normalisers in one exchange per node: block b finds its maximum m_b, its entries' local weights
// e_i = exp((l_i - m_b) * (1/T)) (all zero if m_b = -inf) and their sum s_b, and the exchange hands every block every
// (m_b, s_b).  With M = max m_b and f_b = exp((m_b - M) * (1/T)): Z = sum over b of s_b * f_b in block order, the
// probability of entry i of block b is p_i = e_i * (f_b / Z), and a bonus draw takes the weights e_i * f_b with block
// partials s_b * f_b.
//
// Residual after j >= 1 rejections at a node: r_j = max(p - c_j q, 0) / S_j with c_1 = 1, S_j = sum of the numerator,
// c_{j+1} = c_j + S_j -- algebraically the same as replacing p by norm(max(p - q, 0)) after each rejection, but each
// rejection costs one reduction instead of a rewrite of the distribution.  All arithmetic is float64 with explicit
// single roundings (no contraction): d_i = p_i - c * q_i.
constexpr int ACC_NB = 64, ACC_T = 256, ACC_PER = 16;
constexpr int ACC_XW = 6;   // exchange words per block: two doubles (two words each) and two floats
// Tree inputs staged in LDS by every block at the start (one round of independent loads, also from pinned host
// memory): up to ACC_MAX_NODES nodes, ACC_MAX_TRIALS trials and the first ACC_U_LDS uniforms (later ones are read
// where they lie).
constexpr int ACC_MAX_NODES = 64, ACC_MAX_TRIALS = 1024, ACC_U_LDS = 256;

struct AcceptArgs {
    const float *p_logits;   // target logits [nodes][ld]
    const float *q_logits;   // drafter logits [nodes][ld] (rows of nodes with trials)
    int V, ld;
    const int *token;        // [nodes] token of node i (node 0 = root)
    const int *trial_start;  // [nodes] first entry of node i's trials
    const int *n_trials;     // [nodes]
    const int *trials;       // child node index of each trial
    const double *u;         // uniforms, consumed in order
    int n_u;
    double invT;
    unsigned long long *xbuf;   // exchange words [4][ACC_NB][ACC_XW]
    unsigned *err;           // tag_base | 1 if an exchange timed out, tag_base | 2 for a malformed tree (words of
                             // earlier launches carry other tags, so the word is never cleared)
    unsigned tag_base;       // distinct per launch (low 12 bits are the exchange counter)
    int n_nodes, n_trials_total;
    int *out;                // [0] k, [1..k] accepted node ids, [max_depth+1] final token, [max_depth+2] uniforms used,
                             // [max_depth+3] bonus flag
    int max_depth;
    int *host;               // may be NULL: pinned host block written directly: [0] the err word, [1] block 0's
                             // completion tag, [2] the drawing block's tag, [ACC_HOST_OUT ..] a copy of out
    const int *q_row;        // may be NULL: node i's drafter row is q_row[i] (< n_q_rows) instead of i
    int n_q_rows;
};
constexpr int ACC_HOST_OUT = 16;

struct AccShared {
    double tsum[ACC_T];      // thread chunk sums
    double bpart0[ACC_NB], bpart1[ACC_NB];
    float bmax0[ACC_NB], bmax1[ACC_NB];
    double fac0[ACC_NB], fac1[ACC_NB];
    float fred[ACC_T / 64], fred2[ACC_T / 64];
    double tl;
    int found;
    int ok;
};

__device__ __forceinline__ double d_w(float l, float m, double invT) {
    return exp(__dmul_rn(__dsub_rn((double)l, (double)m), invT));
}

// Whether a block of this launch has reported a failure.
__device__ __forceinline__ bool acc_failed(const AcceptArgs &a) {
    const unsigned e = __hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return (e & ~0xfffu) == a.tag_base && (e & 0xfffu) != 0;
}

// All-gather of two doubles (and, with W = ACC_XW, two floats) per block into sh.bpart0 / bpart1 (bmax0 / bmax1).
// Returns false on timeout (every block then stops).
template <int W>
__device__ bool acc_exchange(const AcceptArgs &a, unsigned &ex, double v0, double v1, float f0, float f1,
                             AccShared &sh) {
    static_assert(W == 4 || W == ACC_XW, "two doubles, or two doubles and two floats");
    const unsigned tag = a.tag_base | (ex & 0xfffu);
    unsigned long long *slot = a.xbuf + (size_t)(ex & 3u) * ACC_NB * ACC_XW;
    ++ex;
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned long long b0 = __double_as_longlong(v0), b1 = __double_as_longlong(v1);
        const unsigned long long t = (unsigned long long)tag << 32;
        unsigned long long *w = slot + blockIdx.x * ACC_XW;
        __hip_atomic_store(w + 0, t | (b0 & 0xffffffffull), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(w + 1, t | (b0 >> 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(w + 2, t | (b1 & 0xffffffffull), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(w + 3, t | (b1 >> 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (W == ACC_XW) {
            __hip_atomic_store(w + 4, t | __float_as_uint(f0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(w + 5, t | __float_as_uint(f1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (threadIdx.x == 0) sh.ok = 1;
    __syncthreads();
    if (threadIdx.x < ACC_NB) {
        unsigned long long *w = slot + threadIdx.x * ACC_XW;
        unsigned long long x[W];
        long spins = 0;
        for (;;) {
            bool all = true;
#pragma unroll
            for (int i = 0; i < W; ++i) x[i] = __hip_atomic_load(w + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int i = 0; i < W; ++i) all = all && (unsigned)(x[i] >> 32) == tag;
            if (all) break;
            if (++spins > (1l << 22) || acc_failed(a)) {
                __hip_atomic_store(a.err, a.tag_base | 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                sh.ok = 0;
                break;
            }
        }
        sh.bpart0[threadIdx.x] = __longlong_as_double((long long)((x[0] & 0xffffffffull) | (x[1] << 32)));
        sh.bpart1[threadIdx.x] = __longlong_as_double((long long)((x[2] & 0xffffffffull) | (x[3] << 32)));
        if (W == ACC_XW) {
            sh.bmax0[threadIdx.x] = __uint_as_float((unsigned)x[W == ACC_XW ? 4 : 0]);
            sh.bmax1[threadIdx.x] = __uint_as_float((unsigned)x[W == ACC_XW ? 5 : 0]);
        }
    }
    __syncthreads();
    return sh.ok != 0;
}

// Block sum of the ACC_T thread chunk sums: butterfly inside each wave (lane l adds lane l ^ o for o = 32 .. 1, so
// every lane holds the same value), then the ACC_T / 64 wave sums in wave order.  Also leaves the thread sums in
// sh.tsum for a draw.
__device__ double acc_block_sum(double mine, AccShared &sh) {
    __shared__ double wsum[ACC_T / 64];
    __syncthreads();
    sh.tsum[threadIdx.x] = mine;
    double v = mine;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, SP_WAVE);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int j = 0; j < ACC_T / 64; ++j) t += wsum[j];
    return t;
}

// Block sums / maxima of two values at once (one barrier round for both); no thread sums are kept.
__device__ void acc_block_sum2(double &a, double &b, AccShared &sh) {
    __shared__ double w2[2][ACC_T / 64];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) { a += __shfl_xor(a, o, SP_WAVE); b += __shfl_xor(b, o, SP_WAVE); }
    __syncthreads();
    if ((threadIdx.x & 63) == 0) { w2[0][threadIdx.x >> 6] = a; w2[1][threadIdx.x >> 6] = b; }
    __syncthreads();
    a = 0.0; b = 0.0;
#pragma unroll
    for (int j = 0; j < ACC_T / 64; ++j) { a += w2[0][j]; b += w2[1][j]; }
}

__device__ void acc_block_max2(float &a, float &b, AccShared &sh) {
    a = wave_max(a);
    b = wave_max(b);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) { sh.fred[threadIdx.x >> 6] = a; sh.fred2[threadIdx.x >> 6] = b; }
    __syncthreads();
    a = sh.fred[0]; b = sh.fred2[0];
    for (int j = 1; j < ACC_T / 64; ++j) { a = fmaxf(a, sh.fred[j]); b = fmaxf(b, sh.fred2[j]); }
}

__device__ float acc_block_max(float v, AccShared &sh) {
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh.fred[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = sh.fred[0];
    for (int j = 1; j < ACC_T / 64; ++j) t = fmaxf(t, sh.fred[j]);
    return t;
}

// Inverse-CDF draw over the distributed weights w[] (this thread's chunk; thread chunk sums in sh.tsum, block
// partials in bp).  Three levels, each "first entry whose running sum exceeds the target, else the last positive
// entry": block (every block, redundantly), thread (thread 0 of the owning block), element (the owning thread).
// If no weight is positive at all the token is 0.  Returns the token in the owning block, -1 in the others.
template <int CP>
__device__ int acc_draw(const double *w, int lo, int n, double u, const double *bp, AccShared &sh) {
    double total = 0.0;
    for (int b = 0; b < ACC_NB; ++b) total += bp[b];
    const double target = __dmul_rn(u, total);
    double P = 0.0, Pown = 0.0, Plast = 0.0;
    int owner = -1, blast = 0;
    for (int b = 0; b < ACC_NB; ++b) {
        const double next = P + bp[b];
        if (bp[b] > 0.0) { blast = b; Plast = P; }
        if (target < next) { owner = b; Pown = P; break; }
        P = next;
    }
    if (owner < 0) { owner = blast; Pown = Plast; }
    if ((int)blockIdx.x != owner) return -1;
    const double tb = __dsub_rn(target, Pown);
    __syncthreads();
    if (threadIdx.x == 0) {
        double q = 0.0, qsel = 0.0, qlast = 0.0;
        int tsel = -1, tlast = 0;
        for (int t = 0; t < ACC_T; ++t) {
            const double next = q + sh.tsum[t];
            if (sh.tsum[t] > 0.0) { tlast = t; qlast = q; }
            if (tb < next) { tsel = t; qsel = q; break; }
            q = next;
        }
        if (tsel < 0) { tsel = tlast; qsel = qlast; }
        sh.found = tsel;
        sh.tl = __dsub_rn(tb, qsel);
    }
    __syncthreads();
    const int tsel = sh.found;
    __syncthreads();
    if ((int)threadIdx.x == tsel) {
        const double tl = sh.tl;
        double acc = 0.0;
        int pick = -1, lastpos = -1;
        for (int i = 0; i < CP; ++i) {
            if (i < n) {
                if (w[i] > 0.0) lastpos = lo + i;
                acc += w[i];
                if (acc > tl) { pick = lo + i; break; }
            }
        }
        if (pick < 0) pick = lastpos >= 0 ? lastpos : lo;
        sh.found = pick;
    }
    __syncthreads();
    return sh.found;
}

// Stops every block identically (the condition depends only on the inputs) and reports a malformed tree.
__device__ __forceinline__ bool acc_bad(const AcceptArgs &a) {
    if (blockIdx.x == 0 && threadIdx.x == 0)
        __hip_atomic_store(a.err, a.tag_base | 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return false;
}

__device__ __forceinline__ void acc_put(const AcceptArgs &a, int i, int v) {
    a.out[i] = v;
    if (a.host) a.host[ACC_HOST_OUT + i] = v;
}

// CP >= C: the entries per thread as a compile-time count, so every per-entry loop is straight-line code whose loads
// and exponentials are independent (entries past the thread's n are read from a clamped index and masked).
template <int CP>
__global__ void __launch_bounds__(ACC_T) k_accept_tree(AcceptArgs a) {
    // p - c q products and differences are rounded separately, as the definition writes them (hipcc would otherwise
    // contract them into fused multiply-adds; __dmul_rn / __dsub_rn are plain operators in HIP)
#pragma clang fp contract(off)
    __shared__ AccShared sh;
    __shared__ int s_token[ACC_MAX_NODES], s_tstart[ACC_MAX_NODES], s_ntr[ACC_MAX_NODES], s_trials[ACC_MAX_TRIALS];
    __shared__ int s_qrow[ACC_MAX_NODES];
    __shared__ double s_u[ACC_U_LDS];
    const int C = (a.V + ACC_NB * ACC_T - 1) / (ACC_NB * ACC_T);
    const int lo = (blockIdx.x * ACC_T + threadIdx.x) * C;
    const int n = max(0, min(C, a.V - lo));
    // the tree and the uniforms into LDS (independent loads, all in flight together)
    for (int i = threadIdx.x; i < a.n_nodes; i += ACC_T) {
        s_token[i] = a.token[i];
        s_tstart[i] = a.trial_start[i];
        s_ntr[i] = a.n_trials[i];
        s_qrow[i] = a.q_row ? a.q_row[i] : i;
    }
    for (int i = threadIdx.x; i < a.n_trials_total; i += ACC_T) s_trials[i] = a.trials[i];
    for (int i = threadIdx.x; i < min(a.n_u, ACC_U_LDS); i += ACC_T) s_u[i] = a.u[i];
    __syncthreads();
    auto uni = [&](int i) { return i < a.n_u ? (i < ACC_U_LDS ? s_u[i] : a.u[i]) : 0.5; };
    double wp[CP], w[CP];
    unsigned ex = 0;
    int cur = 0, k = 0, ui = 0, final_tok = -1, bonus = 0;
    bool alive = true;
    for (;;) {
        const float *pl = a.p_logits + (size_t)cur * a.ld;
        const int nt = s_ntr[cur];
        const int t0 = s_tstart[cur];
        if (nt < 0 || t0 < 0 || t0 > a.n_trials_total - nt) { alive = acc_bad(a); break; }
        for (int j = t0; j < t0 + nt && alive; ++j) {
            const int child = s_trials[j];
            if (child <= 0 || child >= a.n_nodes || s_token[child] < 0 || s_token[child] >= a.V) alive = acc_bad(a);
        }
        const int qr = s_qrow[cur];
        if (nt > 0 && a.q_row && (qr < 0 || qr >= a.n_q_rows)) alive = acc_bad(a);
        if (!alive) break;
        const bool draw_bonus = nt == 0 || k >= a.max_depth;
        const float *ql = a.q_logits + (size_t)(nt > 0 ? qr : 0) * a.ld;
        // the first trial's logits, loaded with the rows (the tree was validated above)
        const int x0 = nt > 0 ? s_token[s_trials[t0]] : 0;
        const float lpx0 = pl[x0], lqx0 = ql[x0];
        // ---- the node's logits (one batch of loads, clamped indices), this block's maxima, its local weights
        // e_i = exp((l_i - m_b) / T) (zero in a block without a finite logit) and their block sums s_b; one exchange
        // of (s_b, m_b) for p and q
        float lp[CP], lq[CP];
#pragma unroll
        for (int i = 0; i < CP; ++i) {
            const int kk = min(lo + i, a.V - 1);
            lp[i] = pl[kk];
            lq[i] = ql[kk];
        }
        float mp = -INFINITY, mq = -INFINITY;
#pragma unroll
        for (int i = 0; i < CP; ++i) {
            if (i < n) { mp = fmaxf(mp, lp[i]); mq = fmaxf(mq, lq[i]); }
        }
        if (draw_bonus) mq = -INFINITY;
        acc_block_max2(mp, mq, sh);
        const bool livep = mp > -INFINITY, liveq = mq > -INFINITY;
        double ep[CP], eq[CP];
#pragma unroll
        for (int i = 0; i < CP; ++i) ep[i] = livep ? d_w(lp[i], mp, a.invT) : 0.0;
        if (!draw_bonus) {
#pragma unroll
            for (int i = 0; i < CP; ++i) eq[i] = liveq ? d_w(lq[i], mq, a.invT) : 0.0;
        }
        double sp = 0.0, sq = 0.0;
#pragma unroll
        for (int i = 0; i < CP; ++i) {
            if (i < n) {
                sp += ep[i];
                if (!draw_bonus) sq += eq[i];
            }
        }
        acc_block_sum2(sp, sq, sh);
        if (!(alive = acc_exchange<ACC_XW>(a, ex, sp, sq, mp, mq, sh))) break;
        float Mp = -INFINITY, Mq = -INFINITY;
        for (int b = 0; b < ACC_NB; ++b) { Mp = fmaxf(Mp, sh.bmax0[b]); Mq = fmaxf(Mq, sh.bmax1[b]); }
        // factors f_b = exp((m_b - M) / T) of the global maxima and the block partials s_b * f_b (thread b, block b)
        if (threadIdx.x < ACC_NB) {
            const int b = threadIdx.x;
            const double fp = d_w(sh.bmax0[b], Mp, a.invT);
            sh.fac0[b] = fp;
            sh.bpart0[b] = __dmul_rn(sh.bpart0[b], fp);
            if (!draw_bonus) {
                const double fq = d_w(sh.bmax1[b], Mq, a.invT);
                sh.fac1[b] = fq;
                sh.bpart1[b] = __dmul_rn(sh.bpart1[b], fq);
            }
        }
        __syncthreads();
        if (draw_bonus) {
            // weights e_i * f_b; thread chunk sums into sh.tsum, block partials s_b * f_b in sh.bpart0
            const double f = sh.fac0[blockIdx.x];
            sp = 0.0;
#pragma unroll
            for (int i = 0; i < CP; ++i) {
                wp[i] = i < n ? __dmul_rn(ep[i], f) : 0.0;
                if (i < n) sp += wp[i];
            }
            (void)acc_block_sum(sp, sh);
            final_tok = acc_draw<CP>(wp, lo, n, uni(ui), sh.bpart0, sh);
            ++ui;
            bonus = 1;
            break;
        }
        double Zp = 0.0, Zq = 0.0;
        for (int b = 0; b < ACC_NB; ++b) { Zp += sh.bpart0[b]; Zq += sh.bpart1[b]; }
        // ---- trials in draw order, with p_i = e_i * (f_b / Zp) and q_i likewise (formed only after a rejection)
        const double gp = __ddiv_rn(sh.fac0[blockIdx.x], Zp), gq = __ddiv_rn(sh.fac1[blockIdx.x], Zq);
        const int span = ACC_T * C;     // entries per block
        int accepted = -1, J = 0;
        double c = 0.0, S = 0.0;
        for (int j = t0; j < t0 + nt; ++j) {
            const int child = s_trials[j];
            const int x = s_token[child];
            const int bx = x / span;
            const float mpx = sh.bmax0[bx], mqx = sh.bmax1[bx];
            float lpx = lpx0, lqx = lqx0;
            if (j != t0) { lpx = pl[x]; lqx = ql[x]; }
            const double px0 = mpx > -INFINITY ? __dmul_rn(d_w(lpx, mpx, a.invT), __ddiv_rn(sh.fac0[bx], Zp)) : 0.0;
            const double qx = mqx > -INFINITY ? __dmul_rn(d_w(lqx, mqx, a.invT), __ddiv_rn(sh.fac1[bx], Zq)) : 0.0;
            double px = px0;
            if (J > 0) {
                const double dx = __dsub_rn(px0, __dmul_rn(c, qx));
                px = dx > 0.0 ? __ddiv_rn(dx, S) : 0.0;
            }
            const double uu = uni(ui);
            ++ui;
            if (uu < __ddiv_rn(px, qx)) { accepted = child; break; }
            // rejection: next residual numerator max(p - c q, 0) with c = 1 (first) or c + S
            c = J == 0 ? 1.0 : c + S;
            ++J;
            double sr = 0.0;
#pragma unroll
            for (int i = 0; i < CP; ++i) {
                const double d = __dsub_rn(__dmul_rn(ep[i], gp), __dmul_rn(c, __dmul_rn(eq[i], gq)));
                w[i] = (i < n && d > 0.0) ? d : 0.0;
            }
#pragma unroll
            for (int i = 0; i < CP; ++i)
                if (i < n) sr += w[i];
            // leaves this residual's thread chunk sums in sh.tsum for a possible final draw
            const double bsr = acc_block_sum(sr, sh);
            if (!(alive = acc_exchange<4>(a, ex, bsr, 0.0, 0.f, 0.f, sh))) break;
            S = 0.0;
            for (int b = 0; b < ACC_NB; ++b) S += sh.bpart0[b];
        }
        if (!alive) break;
        if (accepted >= 0) {
            if (blockIdx.x == 0 && threadIdx.x == 0) acc_put(a, 1 + k, accepted);
            ++k;
            cur = accepted;
            continue;
        }
        // every trial rejected: draw from the last residual (weights w, block partials in sh.bpart0)
        final_tok = acc_draw<CP>(w, lo, n, uni(ui), sh.bpart0, sh);
        ++ui;
        break;
    }
    if (alive && threadIdx.x == 0) {
        if (blockIdx.x == 0) {          // every block took the same decisions; block 0 reports them
            acc_put(a, 0, k);
            for (int i = 1 + k; i <= a.max_depth; ++i) acc_put(a, i, -1);   // unused path entries
            acc_put(a, a.max_depth + 2, ui);
            acc_put(a, a.max_depth + 3, bonus);
        }
        if (final_tok >= 0) acc_put(a, a.max_depth + 1, final_tok);   // only the block owning the draw has it
    }
    // host read-back without a copy or a stream synchronisation: each writer's entries reach host memory before its
    // tag (system-scope fence); the host waits for block 0's tag and, unless the err word reports a failure, for the
    // drawing block's
    if (threadIdx.x == 0 && a.host) {
        if (alive && final_tok >= 0) {
            __threadfence_system();
            __hip_atomic_store(a.host + 2, (int)a.tag_base, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        if (blockIdx.x == 0) {
            a.host[0] = (int)__hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __threadfence_system();
            __hip_atomic_store(a.host + 1, (int)a.tag_base, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Filtered sampling: temperature, top-k and top-p (nucleus) exactly as Qwen2Engine.sample defines them
// (qwen_engine.py:146-156; native Sampler::distribution, sampler.hpp:22-57), many blocks of FS_THREADS per draw.
//   z_i   = fp32(l_i / T);  the order is z descending, ties by ascending index (the native sampler's comparator);
//   top-k (0 < k < V): keep z_i >= the k-th largest z (ties at the cutoff kept);
//   mass  m_i = floor(exp(z_i - z_max) * 2^40) as a 64-bit integer (fp64 exp; z_max = the row maximum, so m <= 2^40
//         and a row sum stays below 2^58): sums are exact and independent of order, so the kernel needs no fixed
//         summation tree; the 2^-40 quantum is far below any probability the cut or the draw can resolve;
//   top-p (p < 1): with F the total mass of the kept tokens, keep the sorted prefix whose exclusive cumulative mass
//         is <= floor(p * F) (first index whose inclusive mass exceeds that, and everything before it);
//   draw: target = floor(u * K) (clamped below K) over the kept mass K; the token is the first in sorted order whose
//         inclusive cumulative mass exceeds the target (inverse CDF, Sampler::draw, sampler.hpp:93-97).
// Selections in sorted order never sort: a radix descent over the 32-bit order key (8 bits per level, LDS histograms
// of counts and 64-bit masses restricted to the candidates, added into global histograms) finds the bin holding the
// k-th token / the target mass; at the last level the bin is one z value, whose tokens (equal masses) are ordered
// by index.
constexpr int FS_THREADS = 1024;

__device__ __forceinline__ uint32_t fs_key(float z) {      // monotone: larger z, larger key
    const uint32_t b = __float_as_uint(z);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float fs_unkey(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
__device__ __forceinline__ unsigned long long fs_mass(float z, float zmax) {
    return (unsigned long long)(exp((double)z - (double)zmax) * 1099511627776.0);    // 2^40
}

struct FsShared {
    unsigned long long hmass[256];
    unsigned int hcnt[256];
    unsigned int hidx[256];             // last level: the smallest index in each bin
    unsigned long long h1mass[256];     // first-level (top 8 key bits) histogram of the candidates, built once
    unsigned int h1cnt[256];
    unsigned long long red64[FS_THREADS / 64];
    unsigned int redu[FS_THREADS / 64];
    unsigned int sel_bin;
    unsigned long long above;
    unsigned int scan[FS_THREADS];
};

// Histogram add with the wave's lanes combined per bin first: most keys of a row share their top bits, and 64 lanes
// adding to one LDS word serialise.  Up to FS_AGG distinct bins of the wave are combined (one atomic per bin, from
// the lowest active lane); lanes left after that add on their own.  Integer sums: the result is order-independent.
#ifndef SP_FS_AGG
#define SP_FS_AGG 1
#endif
constexpr int FS_AGG = SP_FS_AGG;
template <bool MASS>
__device__ __forceinline__ void fs_hist_add(FsShared &sh, bool act, int bin, unsigned long long mass) {
    const int lane = threadIdx.x & 63;
    for (int it = 0; it < FS_AGG; ++it) {
        const unsigned long long pend = __ballot(act);
        if (pend == 0) return;
        const int leader = __ffsll((long long)pend) - 1;
        const int lb = __shfl(bin, leader);
        const bool mine = act && bin == lb;
        const unsigned long long mm = __ballot(mine);
        if constexpr (MASS) {
            unsigned long long v = mine ? mass : 0ull;
            for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
            if (lane == leader) atomicAdd(&sh.hmass[lb], v);
        }
        if (lane == leader) atomicAdd(&sh.hcnt[lb], (unsigned)__popcll(mm));
        act = act && !mine;
    }
    if (act) {
        if constexpr (MASS) atomicAdd(&sh.hmass[bin], mass);
        atomicAdd(&sh.hcnt[bin], 1u);
    }
}

// Inclusive prefix sums over the 64 lanes of a wave.
template <typename I>
__device__ __forceinline__ I fs_wave_scan(I v) {
    const int lane = threadIdx.x & 63;
    for (int o = 1; o < 64; o <<= 1) {
        const I t = __shfl_up(v, o);
        if (lane >= o) v += t;
    }
    return v;
}

// Bin choice of one radix level, by wave 0 (bins in descending order, 4 per lane: lane l holds 255 - 4l - j).
// MASS: the first bin at which above + (mass of the bins before it, inclusive) exceeds `target`; sh.above = the mass
// before that bin.  !MASS: the first bin at which the running count reaches `rem`; sh.redu[0] = rem minus the count
// before it.  Same choice as walking the bins one by one from 255 down.
template <bool MASS>
__device__ __forceinline__ void fs_choose_bin(FsShared &sh, unsigned long long above, unsigned long long target,
                                              unsigned int rem) {
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    unsigned long long v[4], ls = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int b = 255 - 4 * lane - j;
        v[j] = MASS ? sh.hmass[b] : (unsigned long long)sh.hcnt[b];
        ls += v[j];
    }
    const unsigned long long incl = fs_wave_scan<unsigned long long>(ls);
    const bool hit = MASS ? above + incl > target : incl >= (unsigned long long)rem;
    const unsigned long long m = __ballot(hit);
    const int L = m ? __ffsll((long long)m) - 1 : 63;
    if (lane == L) {
        unsigned long long a = (MASS ? above : 0ull) + (incl - ls);
        int chosen = 255 - 4 * lane - 3;
        bool found = false;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (found) continue;
            const bool take = MASS ? a + v[j] > target : a + v[j] >= (unsigned long long)rem;
            if (take) { chosen = 255 - 4 * lane - j; found = true; }
            else a += v[j];
        }
        if (!found) a -= v[3];     // walked past the lane's last bin: that bin is the choice (the serial walk ends there)
        sh.sel_bin = (unsigned)chosen;
        if (MASS) sh.above = a;
        else sh.redu[0] = rem - (unsigned)a;
    }
}

// Block sum of a 64-bit integer (exact, any order).
__device__ __forceinline__ unsigned long long fs_block_sum(unsigned long long v, FsShared &sh) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh.red64[w] = v;
    __syncthreads();
    unsigned long long t = 0;
    for (int i = 0; i < FS_THREADS / 64; ++i) t += sh.red64[i];
    return t;
}

// Index of the rank-th token (index order) whose key equals `key` (a block-wide scan over contiguous chunks).
__device__ int fs_index_of(const float *row, int V, float T, uint32_t key, unsigned long long rank, FsShared &sh) {
    const int C = (V + FS_THREADS - 1) / FS_THREADS, lo = threadIdx.x * C, hi = min(V, lo + C);
    unsigned int cnt = 0;
    for (int i = lo; i < hi; ++i) cnt += fs_key(__fdiv_rn(row[i], T)) == key;
    // exclusive prefix of the counts over the threads, in thread order: wave scans, then the earlier waves' totals
    const unsigned int incl = fs_wave_scan<unsigned int>(cnt);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 63) sh.scan[w] = incl;
    __syncthreads();
    unsigned long long before = incl - cnt;
    for (int j = 0; j < w; ++j) before += sh.scan[j];
    __shared__ int found;
    if (threadIdx.x == 0) found = -1;
    __syncthreads();
    if (rank >= before && rank < before + cnt) {
        unsigned long long r = rank - before;
        for (int i = lo; i < hi; ++i)
            if (fs_key(__fdiv_rn(row[i], T)) == key) {
                if (r == 0) { found = i; break; }
                --r;
            }
    }
    __syncthreads();
    return found;
}

// ---------------------------------------------------------------------------------------------------------------
// The launches: one block covers FM_SPAN consecutive entries of a row (19 blocks for 151936 entries),
// so every pass over the row runs on the whole chip instead of one CU.  Each launch first repeats the bin choice of
// the previous level (every block from the same global histogram, so every block takes the same choice; block 0
// also records it for the later launches), then histograms its entries into LDS and adds the block's bins to the
// level's global histogram with integer atomics (exact, order-independent).  Launches per draw batch: init, max,
// 4 top-k levels (when top-k applies), the candidates' first level, 3 top-p levels (when top-p applies), 3 draw
// levels, finish.  The scratch (histograms and per-row state) is the library's, one set per device: calls on one
// device must not overlap.
#ifndef SP_FM_U
#define SP_FM_U 8
#endif
constexpr int FM_U = SP_FM_U;                      // entries per thread and pass
constexpr int FM_SPAN = FS_THREADS * FM_U;         // entries of a row per block
constexpr int FM_ROWS = 256;                       // rows per launch sequence (the scratch holds this many)
enum { FM_TOPK = 0, FM_H1 = 4, FM_TOPP = 5, FM_DRAW = 8, FM_NLEV = 11 };
struct FmHist {
    unsigned long long mass[256];
    unsigned int cnt[256];
    unsigned int idx[256];                         // last level: the smallest index in each bin
};
struct FmState {
    unsigned int kmax, kmin;
    unsigned int prefix[FM_NLEV];                  // key bits chosen above the level's shift
    unsigned int rem[4];                           // top-k: tokens still to count inside the prefix
    unsigned long long above[FM_NLEV];             // mass before the prefix (sorted order)
    unsigned long long F, tp, K, tgt;
    int topp;                                      // 1: the top-p cut applies (tp < F)
};
struct FmArgs {
    const float *logits;
    int V, ld;
    const int *rows;
    const double *u;
    float T;
    int top_k;                                     // > 0 and < V: the top-k levels ran
    double top_p;                                  // < 1: the top-p levels ran
    int *out;
    FmHist *hist;                                  // [FM_ROWS][FM_NLEV]
    FmState *st;                                   // [FM_ROWS]
    int row0;                                      // draws row0 .. row0 + gridDim.y - 1 (blockIdx.y = draw - row0)
};

__global__ void __launch_bounds__(256) k_fm_init(FmArgs a) {
    const int r = blockIdx.x;
    unsigned int *h = (unsigned int *)(a.hist + (size_t)r * FM_NLEV);
    constexpr int W = sizeof(FmHist) / 4, IDX0 = (256 * 8 + 256 * 4) / 4;
    for (int i = threadIdx.x; i < FM_NLEV * W; i += blockDim.x) h[i] = (i % W) >= IDX0 ? 0xffffffffu : 0u;
    unsigned int *s = (unsigned int *)(a.st + r);
    for (int i = threadIdx.x; i < (int)(sizeof(FmState) / 4); i += blockDim.x) s[i] = 0u;
}

__global__ void __launch_bounds__(FS_THREADS) k_fm_max(FmArgs a) {
    __shared__ unsigned int red[FS_THREADS / 64];
    const int r = blockIdx.y, i0 = blockIdx.x * FM_SPAN;
    const float *row = a.logits + (size_t)a.rows[a.row0 + r] * a.ld;
    float lv[FM_U];
#pragma unroll
    for (int u = 0; u < FM_U; ++u) {
        const int i = i0 + u * FS_THREADS + threadIdx.x;
        lv[u] = i < a.V ? row[i] : -INFINITY;
    }
    uint32_t k = 0;
#pragma unroll
    for (int u = 0; u < FM_U; ++u) k = max(k, fs_key(__fdiv_rn(lv[u], a.T)));
    for (int o = 32; o > 0; o >>= 1) k = max(k, (uint32_t)__shfl_xor((int)k, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = k;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < FS_THREADS / 64; ++i) k = max(k, red[i]);
        atomicMax(&a.st[r].kmax, k);
    }
}

// The level's global histogram into the block's LDS (counts, and masses for a mass level).
__device__ __forceinline__ void fm_load_hist(FsShared &sh, const FmHist &g, bool mass) {
    for (int b = threadIdx.x; b < 256; b += FS_THREADS) {
        sh.hcnt[b] = g.cnt[b];
        sh.hmass[b] = mass ? g.mass[b] : 0ull;
    }
    __syncthreads();
}
// One choice of fs_choose_bin on the histogram in LDS; every thread gets (bin, above or rem).
template <bool MASS>
__device__ __forceinline__ void fm_choose(FsShared &sh, unsigned long long above, unsigned long long target,
                                          unsigned int rem, unsigned int &bin, unsigned long long &above_out,
                                          unsigned int &rem_out) {
    fs_choose_bin<MASS>(sh, above, target, rem);
    __syncthreads();
    bin = sh.sel_bin;
    above_out = MASS ? sh.above : 0ull;
    rem_out = MASS ? 0u : sh.redu[0];
    __syncthreads();
}
// Adds this block's entries with (key & mask) == prefix (and key >= kmin) to the level's global histogram by key
// byte (key >> shift) & 255: counts, masses (MASS), smallest index per bin (IDX).
template <bool MASS, bool IDX>
__device__ __forceinline__ void fm_pass(const FmArgs &a, FsShared &sh, const float *row, float zmax, uint32_t kmin,
                                        uint32_t mask, uint32_t prefix, int shift, FmHist &g) {
    const int i0 = blockIdx.x * FM_SPAN;
    float lv[FM_U];
#pragma unroll
    for (int u = 0; u < FM_U; ++u) {
        const int i = i0 + u * FS_THREADS + threadIdx.x;
        lv[u] = i < a.V ? row[i] : 0.f;
    }
    for (int b = threadIdx.x; b < 256; b += FS_THREADS) { sh.hmass[b] = 0ull; sh.hcnt[b] = 0u; sh.hidx[b] = 0xffffffffu; }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < FM_U; ++u) {
        const int i = i0 + u * FS_THREADS + threadIdx.x;
        const float z = __fdiv_rn(lv[u], a.T);
        const uint32_t k = fs_key(z);
        const bool act = i < a.V && k >= kmin && (k & mask) == prefix;
        fs_hist_add<MASS>(sh, act, (k >> shift) & 255, MASS && act ? fs_mass(z, zmax) : 0ull);
        if (IDX && act) atomicMin(&sh.hidx[(k >> shift) & 255], (unsigned)i);
    }
    __syncthreads();
    for (int b = threadIdx.x; b < 256; b += FS_THREADS) {
        if (sh.hcnt[b] == 0) continue;
        atomicAdd(&g.cnt[b], sh.hcnt[b]);
        if (MASS) atomicAdd(&g.mass[b], sh.hmass[b]);
        if (IDX) atomicMin(&g.idx[b], sh.hidx[b]);
    }
}
__device__ __forceinline__ uint32_t fm_mask(int shift) { return shift >= 24 ? 0u : 0xffffffffu << (shift + 8); }

// Top-k count level j (shift 24 - 8j): the k-th largest key by a radix descent on counts.
__global__ void __launch_bounds__(FS_THREADS) k_fm_topk(FmArgs a, int j) {
    __shared__ FsShared sh;
    const int r = blockIdx.y;
    FmState &S = a.st[r];
    FmHist *H = a.hist + (size_t)r * FM_NLEV;
    const float *row = a.logits + (size_t)a.rows[a.row0 + r] * a.ld;
    uint32_t prefix = 0, rem = (unsigned)a.top_k;
    if (j > 0) {
        fm_load_hist(sh, H[FM_TOPK + j - 1], false);
        unsigned int bin, rn;
        unsigned long long ab;
        fm_choose<false>(sh, 0ull, 0ull, S.rem[j - 1], bin, ab, rn);
        prefix = S.prefix[FM_TOPK + j - 1] | (bin << (32 - 8 * j));
        rem = rn;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) { S.prefix[FM_TOPK + j] = prefix; S.rem[j] = rem; }
    const int shift = 24 - 8 * j;
    fm_pass<false, false>(a, sh, row, 0.f, 0u, fm_mask(shift), prefix, shift, H[FM_TOPK + j]);
}

// The candidates' first level (count and mass by the top key byte), after the top-k cut.
__global__ void __launch_bounds__(FS_THREADS) k_fm_h1(FmArgs a) {
    __shared__ FsShared sh;
    const int r = blockIdx.y;
    FmState &S = a.st[r];
    FmHist *H = a.hist + (size_t)r * FM_NLEV;
    const float *row = a.logits + (size_t)a.rows[a.row0 + r] * a.ld;
    uint32_t kmin = 0;
    if (a.top_k > 0 && a.top_k < a.V) {
        fm_load_hist(sh, H[FM_TOPK + 3], false);
        unsigned int bin, rn;
        unsigned long long ab;
        fm_choose<false>(sh, 0ull, 0ull, S.rem[3], bin, ab, rn);
        kmin = S.prefix[FM_TOPK + 3] | bin;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) S.kmin = kmin;
    fm_pass<true, false>(a, sh, row, fs_unkey(S.kmax), kmin, 0u, 0u, 24, H[FM_H1]);
}

// Total mass F of the candidates (sum of the first-level bins).
__device__ __forceinline__ unsigned long long fm_total(FsShared &sh, const FmHist &h1) {
    unsigned long long f = 0;
    for (int b = threadIdx.x; b < 256; b += FS_THREADS) f += h1.mass[b];
    return fs_block_sum(f, sh);
}

// Mass-selection level j (shift 16 - 8j) of the top-p cut (DRAW false) or of the draw (DRAW true).
template <bool DRAW>
__global__ void __launch_bounds__(FS_THREADS) k_fm_select(FmArgs a, int j) {
    __shared__ FsShared sh;
    const int r = blockIdx.y;
    FmState &S = a.st[r];
    FmHist *H = a.hist + (size_t)r * FM_NLEV;
    const float *row = a.logits + (size_t)a.rows[a.row0 + r] * a.ld;
    const float zmax = fs_unkey(S.kmax);
    const int base = DRAW ? FM_DRAW : FM_TOPP;
    const bool lead = blockIdx.x == 0 && threadIdx.x == 0;
    unsigned long long target, above;
    uint32_t prefix;
    unsigned int bin, rn;
    if (j == 0) {
        if (!DRAW) {
            const unsigned long long F = fm_total(sh, H[FM_H1]);
            const unsigned long long tp = (unsigned long long)(a.top_p * (double)F);
            const int on = tp < F;
            if (lead) { S.F = F; S.tp = tp; S.topp = on; }
            if (!on) return;
            target = tp;
        } else {
            // the kept mass K: the top-p cut's result when it applied, else the candidates' total
            unsigned long long K;
            if (a.top_p < 1.0 && S.topp) {
                fm_load_hist(sh, H[FM_TOPP + 2], true);
                fm_choose<true>(sh, S.above[FM_TOPP + 2], S.tp, 0u, bin, above, rn);
                const uint32_t key = S.prefix[FM_TOPP + 2] | bin;
                const unsigned long long m = fs_mass(fs_unkey(key), zmax);
                const unsigned long long rank = m > 0 ? (S.tp - above) / m : 0;
                K = above + (rank + 1) * m;
            } else {
                K = a.top_p < 1.0 ? S.F : fm_total(sh, H[FM_H1]);
            }
            unsigned long long tgt = (unsigned long long)(a.u[a.row0 + r] * (double)K);
            if (tgt >= K) tgt = K - 1;
            if (lead) { S.K = K; S.tgt = tgt; }
            target = tgt;
        }
        fm_load_hist(sh, H[FM_H1], true);
        fm_choose<true>(sh, 0ull, target, 0u, bin, above, rn);
        prefix = bin << 24;
    } else {
        if (!DRAW && !S.topp) return;
        target = DRAW ? S.tgt : S.tp;
        fm_load_hist(sh, H[base + j - 1], true);
        fm_choose<true>(sh, S.above[base + j - 1], target, 0u, bin, above, rn);
        prefix = S.prefix[base + j - 1] | (bin << (24 - 8 * j));
    }
    if (lead) { S.prefix[base + j] = prefix; S.above[base + j] = above; }
    const int shift = 16 - 8 * j;
    if (shift == 0) fm_pass<true, true>(a, sh, row, zmax, S.kmin, fm_mask(0), prefix, 0, H[base + j]);
    else fm_pass<true, false>(a, sh, row, zmax, S.kmin, fm_mask(shift), prefix, shift, H[base + j]);
}

// The drawn token: the last draw level's choice, its rank inside the tie group, and its index.
__global__ void __launch_bounds__(FS_THREADS) k_fm_finish(FmArgs a) {
    __shared__ FsShared sh;
    const int r = blockIdx.x;
    FmState &S = a.st[r];
    FmHist *H = a.hist + (size_t)r * FM_NLEV;
    const float *row = a.logits + (size_t)a.rows[a.row0 + r] * a.ld;
    const float zmax = fs_unkey(S.kmax);
    fm_load_hist(sh, H[FM_DRAW + 2], true);
    unsigned int bin, rn;
    unsigned long long above;
    fm_choose<true>(sh, S.above[FM_DRAW + 2], S.tgt, 0u, bin, above, rn);
    const uint32_t key = S.prefix[FM_DRAW + 2] | bin;
    const unsigned long long m = fs_mass(fs_unkey(key), zmax);
    const unsigned long long rank = m > 0 ? (S.tgt - above) / m : 0;
    // rank 0 (always, unless the drawn z value is shared by several tokens) is the group's smallest index
    const int tok = rank == 0 ? (int)H[FM_DRAW + 2].idx[key & 255] : fs_index_of(row, a.V, a.T, key, rank, sh);
    if (threadIdx.x == 0) a.out[a.row0 + r] = tok;
}
