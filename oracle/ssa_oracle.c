/*
 * ssa_oracle.c -- CPU restatement of the SSA SparseAttention forward hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product (ssa_amd/) never links, imports or calls it.
 *
 * Every function restates one piece of the reference's algorithm
 * (sparse_attention.py of daedalus/SSA) and cites the lines it follows.  The
 * reference delegates three decisions to library routines whose exact
 * behaviour fixes the output bits; they are restated here from the published
 * algorithms (Musser's introsort / introselect as shipped by libstdc++ 11):
 *
 *   torch.sort(stable=False) on CPU  == std::sort over (key, position) pairs
 *                                       compared on key only
 *   torch.topk(largest, sorted) CPU  == std::nth_element(k-1) + std::sort of
 *                                       the first k-1 (when 64*k > n), else
 *                                       std::partial_sort, comparator
 *                                       "NaN first, then >"
 *   small argsort (<= 16 elements)   == stable insertion order
 *
 * Those equivalences are pinned by tests against torch itself (the library the
 * reference calls), not assumed.
 *
 * Parity status of each function is stated in its comment ("pinned by ...").
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Generic element and comparators                                          */
/* ------------------------------------------------------------------------ */

typedef struct {
    int64_t key;   /* sort key (bucket id) for the permutation sort          */
    float   val;   /* score for the top-k emulation                          */
    int64_t pos;   /* payload: original position                             */
} elem_t;

typedef int (*less_fn)(const elem_t *a, const elem_t *b);

/* Planted mistakes, for the tests that show each pinning check catches one
 * (0 = the faithful restatement).  Never set outside those tests. */
static int g_mut = 0;
void ssa_oracle_set_mutation(int m) { g_mut = m; }
enum {
    MUT_STABLE_SORT = 1,     /* stable sort instead of introsort               */
    MUT_FILLER_NO_MARK = 2,  /* invalid slots do not mark their key as seen    */
    MUT_SIGN_GE = 3,         /* bit = proj >= 0                                */
    MUT_NO_CAUSAL = 4,       /* no causal substitution of future keys          */
    MUT_NO_EMPTY_FB = 5,     /* no glob ++ 0 list for an empty bucket          */
    MUT_NEGINF_ZERO = 6,     /* -inf slots become 0 instead of glob[t]         */
    MUT_PROBE_CUMUL = 7,     /* probe t flips bits cumulatively                */
    MUT_ONE_TOPK = 8,        /* one top-k over the whole row, not chunked      */
    MUT_MERGE_SELF = 9       /* merge keeps the query itself in the pool       */
};

/* key-only '<' : torch.sort(int64) ascending, sparse_attention.py:781 */
static int less_key(const elem_t *a, const elem_t *b) { return a->key < b->key; }

/* torch.topk(largest=True) comparator: NaN ranks first, then '>' */
static int less_topk(const elem_t *a, const elem_t *b) {
    int an = isnan(a->val), bn = isnan(b->val);
    return (an && !bn) || (a->val > b->val);
}

static inline void eswap(elem_t *a, elem_t *b) { elem_t t = *a; *a = *b; *b = t; }

static int floor_log2(long n) { int r = 0; while (n > 1) { n >>= 1; ++r; } return r; }

/* Median of three (a, b, c) moved into *res: the pivot selection rule of
 * libstdc++'s introsort (median of first+1, middle, last-1). */
static void median3_to_front(elem_t *res, elem_t *a, elem_t *b, elem_t *c, less_fn lt) {
    if (lt(a, b)) {
        if (lt(b, c)) eswap(res, b);
        else if (lt(a, c)) eswap(res, c);
        else eswap(res, a);
    } else if (lt(a, c)) {
        eswap(res, a);
    } else if (lt(b, c)) {
        eswap(res, c);
    } else {
        eswap(res, b);
    }
}

/* Hoare partition around *piv without bounds checks; the median-of-three
 * guarantees a stopper on each side.  Returns the cut. */
static elem_t *hoare(elem_t *lo, elem_t *hi, elem_t *piv, less_fn lt) {
    for (;;) {
        while (lt(lo, piv)) ++lo;
        --hi;
        while (lt(piv, hi)) --hi;
        if (!(lo < hi)) return lo;
        eswap(lo, hi);
        ++lo;
    }
}

static elem_t *partition_pivot(elem_t *f, elem_t *l, less_fn lt) {
    elem_t *mid = f + (l - f) / 2;
    median3_to_front(f, f + 1, mid, l - 1, lt);
    return hoare(f + 1, l, f, lt);
}

/* Binary max-heap helpers (hole-sifting variant: sink the hole to a leaf
 * preferring the right child unless it is smaller than the left, then bubble
 * the carried value up). */
static void heap_push_up(elem_t *base, long hole, long top, elem_t v, less_fn lt) {
    long parent = (hole - 1) / 2;
    while (hole > top && lt(&base[parent], &v)) {
        base[hole] = base[parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    base[hole] = v;
}

static void heap_adjust(elem_t *base, long hole, long len, elem_t v, less_fn lt) {
    const long top = hole;
    long child = hole;
    while (child < (len - 1) / 2) {
        child = 2 * (child + 1);
        if (lt(&base[child], &base[child - 1])) child--;
        base[hole] = base[child];
        hole = child;
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
        child = 2 * (child + 1);
        base[hole] = base[child - 1];
        hole = child - 1;
    }
    heap_push_up(base, hole, top, v, lt);
}

static void heap_make(elem_t *f, elem_t *l, less_fn lt) {
    long len = l - f;
    if (len < 2) return;
    long parent = (len - 2) / 2;
    for (;;) {
        elem_t v = f[parent];
        heap_adjust(f, parent, len, v, lt);
        if (parent == 0) return;
        parent--;
    }
}

/* move the top to *res and re-heap [f, l) with the old *res value */
static void heap_pop_into(elem_t *f, elem_t *l, elem_t *res, less_fn lt) {
    elem_t v = *res;
    *res = *f;
    heap_adjust(f, 0, l - f, v, lt);
}

static void heap_select(elem_t *f, elem_t *mid, elem_t *l, less_fn lt) {
    heap_make(f, mid, lt);
    for (elem_t *i = mid; i < l; ++i)
        if (lt(i, f)) heap_pop_into(f, mid, i, lt);
}

static void heap_sort_all(elem_t *f, elem_t *l, less_fn lt) {
    while (l - f > 1) {
        --l;
        heap_pop_into(f, l, l, lt);
    }
}

static void insertion_sort(elem_t *f, elem_t *l, less_fn lt) {
    if (f == l) return;
    for (elem_t *i = f + 1; i != l; ++i) {
        elem_t v = *i;
        if (lt(&v, f)) {
            memmove(f + 1, f, (size_t)(i - f) * sizeof(elem_t));
            *f = v;
        } else {
            elem_t *j = i, *k = i - 1;
            while (lt(&v, k)) { *j = *k; j = k; --k; }
            *j = v;
        }
    }
}

static void unguarded_insertion_sort(elem_t *f, elem_t *l, less_fn lt) {
    for (elem_t *i = f; i != l; ++i) {
        elem_t v = *i;
        elem_t *j = i, *k = i - 1;
        while (lt(&v, k)) { *j = *k; j = k; --k; }
        *j = v;
    }
}

#define SORT_THRESHOLD 16

static void introsort_loop(elem_t *f, elem_t *l, long depth, less_fn lt) {
    while (l - f > SORT_THRESHOLD) {
        if (depth == 0) {
            heap_select(f, l, l, lt);
            heap_sort_all(f, l, lt);
            return;
        }
        --depth;
        elem_t *cut = partition_pivot(f, l, lt);
        introsort_loop(cut, l, depth, lt);
        l = cut;
    }
}

/* std::sort restated: introsort loop with depth limit 2*floor(log2 n), then a
 * final insertion sort (guarded over the first 16, unguarded after). */
static void intro_sort(elem_t *f, elem_t *l, less_fn lt) {
    if (f == l) return;
    introsort_loop(f, l, 2L * floor_log2(l - f), lt);
    if (l - f > SORT_THRESHOLD) {
        insertion_sort(f, f + SORT_THRESHOLD, lt);
        unguarded_insertion_sort(f + SORT_THRESHOLD, l, lt);
    } else {
        insertion_sort(f, l, lt);
    }
}

/* std::nth_element restated (introselect, depth limit 2*floor(log2 n)). */
static void intro_select(elem_t *f, elem_t *nth, elem_t *l, less_fn lt) {
    if (f == l || nth == l) return;
    long depth = 2L * floor_log2(l - f);
    while (l - f > 3) {
        if (depth == 0) {
            heap_select(f, nth + 1, l, lt);
            eswap(f, nth);
            return;
        }
        --depth;
        elem_t *cut = partition_pivot(f, l, lt);
        if (cut <= nth) f = cut; else l = cut;
    }
    insertion_sort(f, l, lt);
}

/* std::partial_sort restated */
static void partial_sort(elem_t *f, elem_t *mid, elem_t *l, less_fn lt) {
    heap_select(f, mid, l, lt);
    heap_sort_all(f, mid, lt);
}

/* ------------------------------------------------------------------------ */
/* Exported: permutation of torch.sort(keys) (unstable)                      */
/*   follows sparse_attention.py:781; pinned by tests against torch.sort     */
/* ------------------------------------------------------------------------ */
void ssa_oracle_sort_perm(const int64_t *keys, long n, int64_t *perm) {
    elem_t *e = (elem_t *)malloc((size_t)(n > 0 ? n : 1) * sizeof(elem_t));
    for (long i = 0; i < n; ++i) { e[i].key = keys[i]; e[i].val = 0.f; e[i].pos = i; }
    if (g_mut == MUT_STABLE_SORT) insertion_sort(e, e + n, less_key);
    else intro_sort(e, e + n, less_key);
    for (long i = 0; i < n; ++i) perm[i] = e[i].pos;
    free(e);
}

/* ------------------------------------------------------------------------ */
/* Exported: torch.topk(vals, k, largest=True, sorted=True) on one row       */
/*   follows the call at sparse_attention.py:921; pinned against torch.topk  */
/* ------------------------------------------------------------------------ */
void ssa_oracle_topk_row(const float *vals, long n, long k, float *out_v, int64_t *out_i) {
    elem_t *e = (elem_t *)malloc((size_t)(n > 0 ? n : 1) * sizeof(elem_t));
    for (long j = 0; j < n; ++j) { e[j].key = 0; e[j].val = vals[j]; e[j].pos = j; }
    if (k > 0) {
        if (k * 64 <= n) {
            partial_sort(e, e + k, e + n, less_topk);
        } else {
            intro_select(e, e + k - 1, e + n, less_topk);
            intro_sort(e, e + k - 1, less_topk);
        }
    }
    for (long j = 0; j < k; ++j) { out_v[j] = e[j].val; out_i[j] = e[j].pos; }
    free(e);
}

/* ------------------------------------------------------------------------ */
/* Small helpers                                                            */
/* ------------------------------------------------------------------------ */

/* fp32 dot in index order; for exact-arithmetic inputs every order agrees */
static float dot_f32(const float *a, const float *b, int d) {
    float s = 0.f;
    for (int i = 0; i < d; ++i) s += a[i] * b[i];
    return s;
}

/* bucket id: bit j = (proj_j > 0), plane j is bit j (sparse_attention.py:589-591) */
static int64_t bucket_of(const float *proj, int P) {
    int64_t id = 0;
    for (int j = 0; j < P; ++j)
        if (g_mut == MUT_SIGN_GE ? proj[j] >= 0.f : proj[j] > 0.f) id |= (int64_t)1 << j;
    return id;
}

/* Probe ids (sparse_attention.py:599-646): order the P planes by |proj|
 * ascending with ties kept in plane order (stable); probe t flips bit order[t]
 * of the BASE id. */
static void probe_ids(const float *proj, int P, int T, int64_t base, int64_t *out) {
    int ord[16];
    for (int j = 0; j < P; ++j) ord[j] = j;
    for (int i = 1; i < P; ++i) {            /* stable insertion by |proj| */
        int v = ord[i], j = i;
        while (j > 0 && fabsf(proj[ord[j - 1]]) > fabsf(proj[v])) { ord[j] = ord[j - 1]; --j; }
        ord[j] = v;
    }
    for (int t = 0; t < T; ++t) {
        int pos = ord[t];
        int bit = (int)((base >> pos) & 1);
        out[t] = base + ((int64_t)1 << pos) * (1 - 2 * bit);
        if (g_mut == MUT_PROBE_CUMUL) base = out[t];
    }
}

/* ------------------------------------------------------------------------ */
/* Exported: per-(row) hash for one round                                    */
/*   proj (rows, P) = x (rows, d) @ planes (P, d)^T in fp32; ids; probe ids  */
/*   follows sparse_attention.py:575-646                                      */
/* ------------------------------------------------------------------------ */
void ssa_oracle_hash(const float *x, long rows, int d, const float *planes, int P, int T,
                     float *proj_out, int64_t *ids_out, int64_t *probes_out) {
    for (long i = 0; i < rows; ++i) {
        float pr[16];
        for (int j = 0; j < P; ++j) pr[j] = dot_f32(x + i * d, planes + (long)j * d, d);
        if (proj_out) memcpy(proj_out + i * P, pr, sizeof(float) * P);
        int64_t id = bucket_of(pr, P);
        ids_out[i] = id;
        if (probes_out && T > 0) probe_ids(pr, P, T, id, probes_out + i * T);
    }
}

/* ------------------------------------------------------------------------ */
/* Exported: LSHGraphBuilder.forward for (BH) independent slices            */
/*                                                                          */
/*   q        (BH, N, d) fp32 (upcast model values)                         */
/*   k        (BK, M, d) fp32; slice bh reads k row block bh / kv_rep        */
/*   q_proj   optional injected (BH, R, N, P) fp32 projections, or NULL      */
/*   k_proj   optional injected (BK, R, M, P) fp32 projections, or NULL      */
/*   planes   (R, maxP, d) fp32 hyperplanes (rand_proj)                      */
/*   glob     (G,) fallback key ids (already clamped by the caller)          */
/*   out_idx  (BH, N, kk) int64, kk = min(top_k, Call)                       */
/*   out_val  optional (BH, N, kk) fp32 selected scores (-inf = fallback)    */
/*   out_tie  optional (BH, N) u8: 1 when the k-th and (k+1)-th finite       */
/*            scores of the final merged row are equal (selection decided by */
/*            the chunked replay's tie order)                                */
/*   out_perm optional (BK, R, M) int64 bucket permutation per round          */
/*                                                                          */
/*   Follows sparse_attention.py:814-959 (forward), 741-810 (_single_round), */
/*   648-739 (_gather_bucket).                                                */
/* ------------------------------------------------------------------------ */
long ssa_oracle_lsh_forward(const float *q, const float *k, long BH, long kv_rep, long N, long M,
                            int d, const float *q_proj, const float *k_proj, const float *planes,
                            int R, int maxP, int P, int T, int C, int top_k, int causal,
                            const int64_t *glob, int G, int64_t *out_idx, float *out_val,
                            uint8_t *out_tie, int64_t *out_perm, long q_step) {
    /* q_step > 1 computes only the query rows n % q_step == 0 (the others are
     * left untouched), for checks at full sizes */
    if (q_step < 1) q_step = 1;
    const int Tp = T < P ? T : P;                        /* :617 min(num_probes, p_eff) */
    const int nsets = 1 + Tp;
    const long Call = (long)R * nsets * C;
    const long kk = top_k < Call ? top_k : Call;         /* :902 */
    long chunk = 4 * kk; if (chunk < 256) chunk = 256; if (chunk > Call) chunk = Call;  /* :903 */
    const long BK = BH / kv_rep;
    const long nb = 1L << P;

    /* per (kv row, round): perm, bucket start / size */
    int64_t *perm = (int64_t *)malloc(sizeof(int64_t) * (size_t)(BK * R * M));
    int64_t *bstart = (int64_t *)malloc(sizeof(int64_t) * (size_t)(BK * R * nb));
    int64_t *bsize = (int64_t *)malloc(sizeof(int64_t) * (size_t)(BK * R * nb));
    int64_t *kid = (int64_t *)malloc(sizeof(int64_t) * (size_t)(M > 0 ? M : 1));
    float *pr = (float *)malloc(sizeof(float) * (size_t)((M > N ? M : N) * P + 1));
    for (long g = 0; g < BK; ++g) {
        for (int r = 0; r < R; ++r) {
            const float *pl = planes + (long)r * maxP * d;
            if (k_proj) {
                const float *kp = k_proj + ((g * R + r) * M) * P;
                for (long m = 0; m < M; ++m) kid[m] = bucket_of(kp + m * P, P);
            } else {
                ssa_oracle_hash(k + g * M * d, M, d, pl, P, 0, pr, kid, NULL);
            }
            int64_t *pm = perm + (g * R + r) * M;
            ssa_oracle_sort_perm(kid, M, pm);                              /* :781 */
            int64_t *bs = bstart + (g * R + r) * nb, *bz = bsize + (g * R + r) * nb;
            for (long u = 0; u < nb; ++u) { bs[u] = M; bz[u] = 0; }       /* :785-790 */
            for (long p = 0; p < M; ++p) {                                  /* :791-792 */
                int64_t u = kid[pm[p]];
                if (p < bs[u]) bs[u] = p;
                bz[u]++;
            }
        }
    }
    if (out_perm) memcpy(out_perm, perm, sizeof(int64_t) * (size_t)(BK * R * M));

    /* per-query stream buffers */
    int64_t *cand = (int64_t *)malloc(sizeof(int64_t) * (size_t)(Call > 0 ? Call : 1));
    uint8_t *valid = (uint8_t *)malloc((size_t)(Call > 0 ? Call : 1));
    int64_t *stamp = (int64_t *)malloc(sizeof(int64_t) * (size_t)(M > 0 ? M : 1));
    int64_t *qids = (int64_t *)malloc(sizeof(int64_t) * (size_t)(R * nsets));
    float *tv = (float *)malloc(sizeof(float) * (size_t)(kk + 1));
    int64_t *ti = (int64_t *)malloc(sizeof(int64_t) * (size_t)(kk + 1));
    float *bestv = (float *)malloc(sizeof(float) * (size_t)(kk + 1));
    int64_t *besti = (int64_t *)malloc(sizeof(int64_t) * (size_t)(kk + 1));
    float *mv = (float *)malloc(sizeof(float) * (size_t)(kk + Call + 1));
    int64_t *mi = (int64_t *)malloc(sizeof(int64_t) * (size_t)(kk + Call + 1));
    float *scores = (float *)malloc(sizeof(float) * (size_t)(Call > 0 ? Call : 1));
    long n_ties = 0;

    for (long bh = 0; bh < BH; ++bh) {
        const long g = bh / kv_rep;
        const float *kg = k + g * M * d;
        for (long m = 0; m < M; ++m) stamp[m] = -1;
        for (long n = 0; n < N; n += q_step) {
            const float *qn = q + (bh * N + n) * d;
            /* id sets per round: primary then probes (:793-795) */
            for (int r = 0; r < R; ++r) {
                float pq[16];
                if (q_proj) {
                    memcpy(pq, q_proj + ((bh * R + r) * N + n) * P, sizeof(float) * P);
                } else {
                    const float *pl = planes + (long)r * maxP * d;
                    for (int j = 0; j < P; ++j) pq[j] = dot_f32(qn, pl + (long)j * d, d);
                }
                int64_t base = bucket_of(pq, P);
                qids[r * nsets] = base;
                if (Tp > 0) probe_ids(pq, P, Tp, base, qids + r * nsets + 1);
            }
            /* candidate stream in concatenation order (:869-877) */
            long j = 0;
            for (int r = 0; r < R; ++r) {
                const int64_t *pm = perm + (g * R + r) * M;
                const int64_t *bs = bstart + (g * R + r) * nb, *bz = bsize + (g * R + r) * nb;
                for (int t = 0; t < nsets; ++t) {
                    int64_t u = qids[r * nsets + t];
                    int64_t st = bs[u], sz = bz[u];
                    int64_t bend = st + sz - 1; if (bend > M - 1) bend = M - 1;   /* :676 */
                    for (int c = 0; c < C; ++c, ++j) {
                        int64_t p = st + c;
                        int v = p <= bend;                                         /* :690 */
                        int64_t gp = v ? p : M; if (gp > M - 1) gp = M - 1;        /* :691-696 */
                        int64_t cv = pm[gp];
                        if (causal && cv > n && g_mut != MUT_NO_CAUSAL) cv = n;    /* :698-709 */
                        if (sz == 0 && g_mut != MUT_NO_EMPTY_FB) {                 /* :711-737 */
                            cv = (c < G) ? glob[c] : 0;
                            v = 1;
                        }
                        cand[j] = cv; valid[j] = (uint8_t)v;
                    }
                }
            }
            /* first occurrence in stream order, regardless of validity (:884-890) */
            const int64_t tag = bh * N + n;
            for (long jj = 0; jj < Call; ++jj) {
                int64_t cv = cand[jj];
                int first = stamp[cv] != tag;
                if (valid[jj] || g_mut != MUT_FILLER_NO_MARK) stamp[cv] = tag;
                int keep = valid[jj] && first;
                scores[jj] = keep ? dot_f32(qn, kg + cv * d, d) : -INFINITY;      /* :909-916 */
            }
            /* chunked running top-k (:904-922) */
            for (long t = 0; t < kk; ++t) { bestv[t] = -INFINITY; besti[t] = 0; }
            const long step = g_mut == MUT_ONE_TOPK ? Call : chunk;
            for (long s0 = 0; s0 < Call; s0 += step) {
                long s1 = s0 + step < Call ? s0 + step : Call;
                long w = kk + (s1 - s0);
                for (long t = 0; t < kk; ++t) { mv[t] = bestv[t]; mi[t] = besti[t]; }
                for (long t = s0; t < s1; ++t) { mv[kk + t - s0] = scores[t]; mi[kk + t - s0] = cand[t]; }
                ssa_oracle_topk_row(mv, w, kk, tv, ti);
                for (long t = 0; t < kk; ++t) { bestv[t] = tv[t]; besti[t] = mi[ti[t]]; }
            }
            /* boundary tie flag: compare k-th selected with the best excluded
             * finite score of the whole row */
            if (out_tie) {
                uint8_t tie = 0;
                float kth = kk > 0 ? bestv[kk - 1] : -INFINITY;
                if (kk > 0 && isfinite(kth)) {
                    /* count finite kept scores equal to kth in the row vs in best */
                    long in_row = 0, in_best = 0;
                    for (long jj = 0; jj < Call; ++jj) if (scores[jj] == kth) in_row++;
                    for (long t = 0; t < kk; ++t) if (bestv[t] == kth) in_best++;
                    tie = in_row > in_best;
                }
                out_tie[bh * N + n] = tie;
                n_ties += tie;
            }
            /* -inf slots -> glob[t] or 0 by slot position (:948-957) */
            int64_t *oi = out_idx + (bh * N + n) * kk;
            for (long t = 0; t < kk; ++t) {
                if (isinf(bestv[t]) && bestv[t] < 0)
                    oi[t] = (t < G && g_mut != MUT_NEGINF_ZERO) ? glob[t] : 0;
                else oi[t] = besti[t];
            }
            if (out_val) memcpy(out_val + (bh * N + n) * kk, bestv, sizeof(float) * (size_t)kk);
        }
    }
    free(perm); free(bstart); free(bsize); free(kid); free(pr); free(cand); free(valid);
    free(stamp); free(qids); free(tv); free(ti); free(bestv); free(besti); free(mv); free(mi); free(scores);
    return n_ties;
}

/* ------------------------------------------------------------------------ */
/* Exported: merge_neighbors (sparse_attention.py:966-1089)                  */
/*   win   (N, Kw) int64 (Kw may be 0)                                       */
/*   glob  (G,) int64                                                        */
/*   lsh   (BH, N, Kl) int64                                                 */
/*   has_self: self index n at slot 0 (self-attention)                       */
/*   out   (BH, N, Kout) int64, valid (BH, N, Kout) u8                       */
/*   Kout = has_self ? 1 + min(total_k-1, Kall) : min(total_k, Kall)          */
/* ------------------------------------------------------------------------ */
static int cmp_i64(const void *a, const void *b) {
    int64_t x = *(const int64_t *)a, y = *(const int64_t *)b;
    return (x > y) - (x < y);
}

void ssa_oracle_merge(const int64_t *win, long Kw, const int64_t *glob, long G, const int64_t *lsh,
                      long Kl, long BH, long N, int has_self, long total_k, int64_t *out,
                      uint8_t *valid) {
    const long Kall = Kw + G + Kl;
    /* true max over the whole combined tensor (:1036) */
    int64_t tmax = INT64_MIN;
    for (long i = 0; i < N * Kw; ++i) if (win[i] > tmax) tmax = win[i];
    if (BH > 0 && N > 0) for (long i = 0; i < G; ++i) if (glob[i] > tmax) tmax = glob[i];
    for (long i = 0; i < BH * N * Kl; ++i) if (lsh[i] > tmax) tmax = lsh[i];
    const int64_t sentinel = tmax + 1;
    long ks = has_self ? (total_k - 1 < Kall ? total_k - 1 : Kall) : (total_k < Kall ? total_k : Kall);
    if (ks < 0) ks = 0;
    const long Kout = has_self ? 1 + ks : ks;
    int64_t *row = (int64_t *)malloc(sizeof(int64_t) * (size_t)(Kall > 0 ? Kall : 1));
    for (long bh = 0; bh < BH; ++bh) {
        for (long n = 0; n < N; ++n) {
            long c = 0;
            for (long i = 0; i < Kw; ++i) row[c++] = win[n * Kw + i];
            for (long i = 0; i < G; ++i) row[c++] = glob[i];
            for (long i = 0; i < Kl; ++i) row[c++] = lsh[(bh * N + n) * Kl + i];
            if (has_self && g_mut != MUT_MERGE_SELF)                         /* :1043-1049 */
                for (long i = 0; i < Kall; ++i) if (row[i] == n) row[i] = sentinel;
            qsort(row, (size_t)Kall, sizeof(int64_t), cmp_i64);              /* :1052 */
            for (long i = Kall - 1; i >= 1; --i)                             /* :1053-1059 */
                if (row[i] == row[i - 1]) row[i] = sentinel;
            qsort(row, (size_t)Kall, sizeof(int64_t), cmp_i64);              /* :1060 */
            int64_t *o = out + (bh * N + n) * Kout;
            uint8_t *vv = valid + (bh * N + n) * Kout;
            long w = 0;
            if (has_self) o[w++] = n;                                        /* :1062-1066 */
            for (long i = 0; i < ks; ++i) o[w++] = row[i];
            for (long i = 0; i < Kout; ++i) {                                /* :1074-1088 */
                vv[i] = o[i] <= tmax;
                if (has_self && i == 0) vv[i] = 1;
                int64_t x = o[i] > tmax ? 0 : o[i];
                if (x < 0) x = 0;
                if (x > tmax) x = tmax;
                o[i] = x;
            }
        }
    }
    free(row);
}

/* ------------------------------------------------------------------------ */
/* Exported: sparse_gather_attention (sparse_attention.py:1096-1199)         */
/*   q (BH,N,d), k/v (BK,M,d) fp32 values of the model tensors; slice bh      */
/*   reads kv block bh / kv_rep; nb (BH,N,K) int64; valid (BH,N,K) u8 or NULL */
/*   mode 0: fp32 model dtype  -> out = sum p*v (double accumulate)           */
/*   mode 1: 16-bit model dtype, p rounded to bf16 before P.V (default path)  */
/*   mode 2: fp16 model dtype, p rounded to fp16 before P.V                   */
/*   fp32w : fp32_attn_weights=True -> p kept in fp32                         */
/*   out (BH,N,d) double (caller rounds to the model dtype)                   */
/* ------------------------------------------------------------------------ */
static float round_bf16(float x) {
    uint32_t u; memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) return x;       /* inf / nan */
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    u &= 0xffff0000u;
    float y; memcpy(&y, &u, 4);
    return y;
}

/* round-to-nearest-even to IEEE binary16 and back (normal, subnormal, overflow) */
static float round_fp16(float x) {
    if (isnan(x) || isinf(x)) return x;
    float ax = fabsf(x);
    if (ax >= 65520.f) return copysignf(INFINITY, x);
    int e;
    frexpf(ax, &e);                       /* ax = m * 2^e, m in [0.5, 1) */
    int ulp_exp = e - 11;                 /* 11 significant bits */
    if (ulp_exp < -24) ulp_exp = -24;     /* subnormal spacing 2^-24 */
    float ulp = ldexpf(1.f, ulp_exp);
    float y = nearbyintf(ax / ulp) * ulp; /* default rounding mode: ties to even */
    return copysignf(y, x);
}

void ssa_oracle_apply(const float *q, const float *k, const float *v, const int64_t *nb,
                      const uint8_t *valid, long BH, long kv_rep, long N, long M, int d, long K,
                      float scale, int mode, int fp32w, double *out) {
    double *s = (double *)malloc(sizeof(double) * (size_t)(K > 0 ? K : 1));
    for (long bh = 0; bh < BH; ++bh) {
        const long g = bh / kv_rep;
        for (long n = 0; n < N; ++n) {
            const float *qn = q + (bh * N + n) * d;
            const int64_t *nn = nb + (bh * N + n) * K;
            double mx = -INFINITY;
            for (long j = 0; j < K; ++j) {
                int ok = valid ? valid[(bh * N + n) * K + j] : 1;
                if (!ok) { s[j] = -INFINITY; continue; }
                const float *kr = k + (g * M + nn[j]) * d;
                double acc = 0.0;
                for (int i = 0; i < d; ++i) acc += (double)qn[i] * (double)kr[i];
                s[j] = acc * (double)scale;
                if (s[j] > mx) mx = s[j];
            }
            double sum = 0.0;
            for (long j = 0; j < K; ++j) { s[j] = isinf(s[j]) ? 0.0 : exp(s[j] - mx); sum += s[j]; }
            double *o = out + (bh * N + n) * d;
            for (int i = 0; i < d; ++i) o[i] = 0.0;
            for (long j = 0; j < K; ++j) {
                double p = s[j] / sum;
                if (!fp32w) {
                    if (mode == 1) p = (double)round_bf16((float)p);
                    else if (mode == 2) p = (double)round_fp16((float)p);
                }
                if (p == 0.0) continue;
                const float *vr = v + (g * M + nn[j]) * d;
                for (int i = 0; i < d; ++i) o[i] += p * (double)vr[i];
            }
        }
    }
    free(s);
}
