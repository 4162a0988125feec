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

constexpr int SMP_THREADS = 1024;

__device__ __forceinline__ double block_sum_d(double v, double *red) {
    // fixed-order: lanes -> waves (butterfly, deterministic for a fixed input) -> sequential over waves
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, SP_WAVE);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = 0.0;
    for (int j = 0; j < (int)(blockDim.x >> 6); ++j) t += red[j];
    return t;
}

__device__ __forceinline__ float block_max_f(float v, float *red) {
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = red[0];
    for (int j = 1; j < (int)(blockDim.x >> 6); ++j) t = fmaxf(t, red[j]);
    return t;
}

// Per-block scratch for the chunked sums.
struct SmpShared {
    double chunk[SMP_THREADS];   // chunk sums, then exclusive prefixes
    double red[16];
    float redf[16];
    double total;
    int found;
};

// Weight of entry i for the distribution being scanned.
//   mode 0: exp((l[i] - m) * invT)                         (unnormalised softmax of `l`)
//   mode 1: r[i]                                           (explicit fp64 weights, the residual)
struct Dist {
    int mode;
    const float *l;
    float m;
    double invT;
    const double *r;
    __device__ __forceinline__ double w(int i) const {
        return mode == 0 ? exp(((double)l[i] - (double)m) * invT) : r[i];
    }
};

// Z = sum of weights in the fixed chunk order; leaves the chunk sums in sh.chunk.
__device__ double dist_total(const Dist &d, int V, SmpShared &sh) {
    const int C = (V + SMP_THREADS - 1) / SMP_THREADS;
    const int lo = threadIdx.x * C, hi = min(V, lo + C);
    double s = 0.0;
    for (int i = lo; i < hi; ++i) s += d.w(i);
    sh.chunk[threadIdx.x] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int j = 0; j < SMP_THREADS; ++j) t += sh.chunk[j];
        sh.total = t;
    }
    __syncthreads();
    return sh.total;
}

// Inverse-CDF draw with target = u * Z (call right after dist_total with the same distribution): the chunk t with
// P_t <= target < P_{t+1} (exclusive prefixes P, the last chunk open above) is scanned from zero against
// target - P_t; the first index whose running sum exceeds it is drawn.  If rounding leaves no such index, the last
// positive-weight index of that chunk is drawn, or else the last positive-weight index of the row.
__device__ int dist_draw(const Dist &d, int V, double u, SmpShared &sh) {
    const int C = (V + SMP_THREADS - 1) / SMP_THREADS;
    __syncthreads();
    if (threadIdx.x == 0) {
        double p = 0.0;
        for (int j = 0; j < SMP_THREADS; ++j) { const double s = sh.chunk[j]; sh.chunk[j] = p; p += s; }
        sh.found = 0x7fffffff;
    }
    __syncthreads();
    const double target = u * sh.total;
    const int t = threadIdx.x;
    const int lo = t * C, hi = min(V, lo + C);
    const double start = sh.chunk[t];
    const bool last = t + 1 == SMP_THREADS;
    if (target >= start && (last || target < sh.chunk[t + 1])) {
        const double tl = target - start;
        double acc = 0.0;
        int pick = -1, lastpos = -1;
        for (int i = lo; i < hi; ++i) {
            const double wi = d.w(i);
            if (wi > 0.0) lastpos = i;
            acc += wi;
            if (acc > tl) { pick = i; break; }
        }
        if (pick < 0) pick = lastpos;
        if (pick >= 0) atomicMin(&sh.found, pick);
    }
    __syncthreads();
    if (sh.found == 0x7fffffff) {
        __syncthreads();
        if (threadIdx.x == 0) {
            int tok = V - 1;
            while (tok > 0 && !(d.w(tok) > 0.0)) --tok;
            sh.found = tok;
        }
        __syncthreads();
    }
    return sh.found;
}

__device__ float row_max(const float *l, int V, SmpShared &sh) {
    float m = -INFINITY;
    for (int i = threadIdx.x; i < V; i += blockDim.x) m = fmaxf(m, l[i]);
    return block_max_f(m, sh.redf);
}

// One block per sample s: out[s] = inverse-CDF draw from softmax(logits[rows[s]] / T) with uniform u[s].
__global__ void __launch_bounds__(SMP_THREADS) k_sample(const float *logits, int V, int ld, const int *rows,
                                                         const double *u, double invT, int *out) {
    __shared__ SmpShared sh;
    const int s = blockIdx.x;
    const float *l = logits + (size_t)rows[s] * ld;
    Dist d{0, l, row_max(l, V, sh), invT, nullptr};
    dist_total(d, V, sh);
    const int tok = dist_draw(d, V, u[s], sh);
    if (threadIdx.x == 0) out[s] = tok;
}

struct AcceptArgs {
    const float *p_logits;   // target logits [nodes][ld]
    const float *q_logits;   // drafter logits [nodes][ld] (rows of nodes with children)
    int V, ld;
    const int *token;        // [nodes] token of node i (node 0 = root)
    const int *trial_start;  // [nodes] first entry of node i's trials
    const int *n_trials;     // [nodes]
    const int *trials;       // child node index of each trial
    const double *u;         // uniforms, consumed in order
    int n_u;
    double invT;
    double *resid;           // scratch [V] fp64
    int *out;                // [0] accepted count k, [1..k] accepted node ids, [max_depth+1] final token,
                             // [max_depth+2] uniforms consumed, [max_depth+3] 1 if final is a bonus draw
    int max_depth;
};

// The whole acceptance walk in one block (it is sequential by nature; every step is a reduction over V).
__global__ void __launch_bounds__(SMP_THREADS) k_accept_tree(AcceptArgs a) {
    __shared__ SmpShared sh;
    int cur = 0, k = 0, ui = 0;
    int final_tok = -1, bonus = 0;
    for (;;) {
        const int nt = a.n_trials[cur];
        const float *pl = a.p_logits + (size_t)cur * a.ld;
        Dist p{0, pl, row_max(pl, a.V, sh), a.invT, nullptr};
        if (nt == 0 || k >= a.max_depth) {                   // bonus draw from the target at the accepted leaf
            dist_total(p, a.V, sh);
            final_tok = dist_draw(p, a.V, ui < a.n_u ? a.u[ui] : 0.5, sh);
            ++ui; bonus = 1;
            break;
        }
        const float *ql = a.q_logits + (size_t)cur * a.ld;
        Dist q{0, ql, row_max(ql, a.V, sh), a.invT, nullptr};
        const double Zq = dist_total(q, a.V, sh);
        double Zp = dist_total(p, a.V, sh);
        bool residual = false;      // p is the explicit normalised residual in a.resid
        int accepted = -1;
        const int t0 = a.trial_start[cur];
        for (int j = t0; j < t0 + nt && accepted < 0; ++j) {
            {
                const int c = a.trials[j];
                const int x = a.token[c];
                const double px = residual ? a.resid[x] : p.w(x) / Zp;
                const double qx = q.w(x) / Zq;
                const double uu = ui < a.n_u ? a.u[ui] : 0.5;
                ++ui;
                if (uu < px / qx) { accepted = c; break; }
                // rejection: p <- norm(max(p - q, 0))
                __syncthreads();
                for (int i = threadIdx.x; i < a.V; i += blockDim.x) {
                    const double pi = residual ? a.resid[i] : p.w(i) / Zp;
                    const double di = pi - q.w(i) / Zq;
                    a.resid[i] = di > 0.0 ? di : 0.0;
                }
                __syncthreads();
                Dist r{1, nullptr, 0.f, 0.0, a.resid};
                const double Zr = dist_total(r, a.V, sh);
                for (int i = threadIdx.x; i < a.V; i += blockDim.x) a.resid[i] = a.resid[i] / Zr;
                __syncthreads();
                residual = true;
            }
        }
        if (accepted >= 0) {
            if (threadIdx.x == 0) a.out[1 + k] = accepted;
            ++k;
            cur = accepted;
            continue;
        }
        // every child rejected: draw from the residual
        Dist r{1, nullptr, 0.f, 0.0, a.resid};
        dist_total(r, a.V, sh);
        final_tok = dist_draw(r, a.V, ui < a.n_u ? a.u[ui] : 0.5, sh);
        ++ui;
        break;
    }
    if (threadIdx.x == 0) {
        a.out[0] = k;
        a.out[a.max_depth + 1] = final_tok;
        a.out[a.max_depth + 2] = ui;
        a.out[a.max_depth + 3] = bonus;
    }
}
