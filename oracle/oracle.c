/*
 * CPU oracle for the semi-naive fixpoint path.  TEST INFRASTRUCTURE ONLY:
 * it is the checker that the GPU library is compared against, used by
 * tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py,
 * never by the product path.
 *
 * It restates, single-threaded and in plain C, the semantics of:
 *   - order / equality of u32 tuples: lexicographic, unsigned per column,
 *     bytewise equality (crates/xlog-cuda/kernels/dedup.cu:293-345,398-404;
 *     LSD order relational.rs:1972-1973).  A tuple (c0, c1) is packed as
 *     (c0 << 32) | c1 so that unsigned u64 order is that order.
 *   - sort (relational.rs:1881-2220), full-row dedup (relational.rs:1558-1677),
 *     union / union_many (relational.rs:822-999), diff (relational.rs:1102-1147,
 *     1311-1428): all set-valued on sorted unique packed keys.
 *   - inner equi-join with output = left columns ++ right columns
 *     (relational.rs:4417-4625) and projection (expression.rs:779-834).
 *   - the semi-naive loop Executor::execute_recursive_scc
 *     (crates/xlog-runtime/src/executor/recursive.rs:447-957): seed pass over
 *     every rule, one variant per recursive scan occurrence with a non-empty
 *     delta (recursive.rs:632-669, rewrite.rs:413-500), delta = (U variants) \ R,
 *     convergence test, merge, iteration count including the final empty
 *     iteration (recursive.rs:619-620,808-865).
 *
 * Independent cross-checks live beside it: a BFS-layer transitive closure
 * (iteration count = max finite shortest-path length) and a naive fixpoint
 * (R <- R U T(R) until stable).
 *
 * or_set_threads(t > 1) switches the sort, the join probe and the BFS to
 * OpenMP versions (used for the multi-core CPU baseline).  They produce the
 * same results as the single-threaded code, which stays the pinned reference
 * for them (tests/test_oracle.py compares both).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <stdio.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;
/* threads for the parallel paths (1 = the single-threaded code) */
int or_set_threads(int t) {
#ifdef _OPENMP
    g_threads = t > 1 ? t : 1;
#else
    (void)t;
    g_threads = 1;
#endif
    return g_threads;
}
int or_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* sorted-vector primitives                                                  */
/* ------------------------------------------------------------------------ */

static int sort_u64_serial(uint64_t *a, uint64_t n);
#ifdef _OPENMP
/* Parallel form: one stable counting pass on the most significant digit that
 * varies (every thread counts its contiguous chunk, offsets digit-major then
 * thread-minor, every thread scatters its chunk in order), then the 256
 * buckets -- whose keys agree on that digit and every digit above it -- are
 * sorted independently by the serial LSD sort, buckets spread over the
 * threads.  The result is the sorted array, as from the serial sort. */
static int sort_u64_mt(uint64_t *a, uint64_t n, int T) {
    uint64_t orv = 0, andv = ~0ull;
    for (uint64_t i = 0; i < n; ++i) { orv |= a[i]; andv &= a[i]; }
    uint64_t diff = orv ^ andv;  /* bits that vary */
    if (!diff) return 0;
    int D = 7;
    while (D > 0 && !((diff >> (8 * D)) & 255)) --D;
    uint64_t *tmp = (uint64_t *)malloc(n * sizeof(uint64_t));
    uint64_t *cnt = (uint64_t *)calloc((size_t)T * 256, sizeof(uint64_t));
    uint64_t bstart[257];
    if (!tmp || !cnt) { free(tmp); free(cnt); return -2; }
    const int sh = 8 * D;
    int rc = 0;
    #pragma omp parallel num_threads(T)
    {
        const int t = omp_get_thread_num();
        const uint64_t lo = n * (uint64_t)t / (uint64_t)T, hi = n * (uint64_t)(t + 1) / (uint64_t)T;
        uint64_t *c = cnt + (size_t)t * 256;
        for (uint64_t i = lo; i < hi; ++i) c[(a[i] >> sh) & 255]++;
        #pragma omp barrier
        #pragma omp single
        {
            uint64_t acc = 0;
            for (int b = 0; b < 256; ++b) {
                bstart[b] = acc;
                for (int u = 0; u < T; ++u) {
                    uint64_t v = cnt[(size_t)u * 256 + b];
                    cnt[(size_t)u * 256 + b] = acc;
                    acc += v;
                }
            }
            bstart[256] = acc;
        }
        for (uint64_t i = lo; i < hi; ++i) {
            uint64_t k = a[i];
            tmp[c[(k >> sh) & 255]++] = k;
        }
        #pragma omp barrier
        #pragma omp for schedule(dynamic, 1)
        for (int b = 0; b < 256; ++b) {
            if (sort_u64_serial(tmp + bstart[b], bstart[b + 1] - bstart[b])) {
                #pragma omp atomic write
                rc = -2;
            }
            memcpy(a + bstart[b], tmp + bstart[b], (bstart[b + 1] - bstart[b]) * sizeof(uint64_t));
        }
    }
    free(tmp); free(cnt);
    return rc;
}
#endif

/* LSD radix sort of u64 keys, 8-bit digits, digits that are constant over
 * the whole input are skipped.  Stable (a textbook counting sort per pass). */
int or_sort_u64(uint64_t *a, uint64_t n) {
    if (n < 2) return 0;
#ifdef _OPENMP
    if (g_threads > 1 && n >= (1u << 16)) return sort_u64_mt(a, n, g_threads);
#endif
    return sort_u64_serial(a, n);
}
static int sort_u64_serial(uint64_t *a, uint64_t n) {
    if (n < 2) return 0;
    uint64_t *tmp = (uint64_t *)malloc(n * sizeof(uint64_t));
    if (!tmp) return -2;
    uint64_t (*cnt)[256] = (uint64_t (*)[256])calloc(8 * 256, sizeof(uint64_t));
    if (!cnt) { free(tmp); return -2; }
    for (uint64_t i = 0; i < n; ++i) {
        uint64_t k = a[i];
        for (int d = 0; d < 8; ++d) cnt[d][(k >> (8 * d)) & 255]++;
    }
    uint64_t *src = a, *dst = tmp;
    for (int d = 0; d < 8; ++d) {
        int trivial = 0;
        for (int b = 0; b < 256; ++b) if (cnt[d][b] == n) { trivial = 1; break; }
        if (trivial) continue;
        uint64_t off[256], acc = 0;
        for (int b = 0; b < 256; ++b) { off[b] = acc; acc += cnt[d][b]; }
        for (uint64_t i = 0; i < n; ++i) {
            uint64_t k = src[i];
            dst[off[(k >> (8 * d)) & 255]++] = k;
        }
        uint64_t *t = src; src = dst; dst = t;
    }
    if (src != a) memcpy(a, src, n * sizeof(uint64_t));
    free(tmp); free(cnt);
    return 0;
}

/* in-place unique of a sorted array; returns the new length */
uint64_t or_unique_sorted(uint64_t *a, uint64_t n) {
    if (n == 0) return 0;
    uint64_t w = 1;
    for (uint64_t i = 1; i < n; ++i) if (a[i] != a[w - 1]) a[w++] = a[i];
    return w;
}

uint64_t or_sort_dedup(uint64_t *a, uint64_t n) {
    if (or_sort_u64(a, n)) return (uint64_t)-1;
    return or_unique_sorted(a, n);
}

/* A \ B for sorted unique A, B; out may alias A.  Returns |out|. */
uint64_t or_diff_sorted(const uint64_t *a, uint64_t na, const uint64_t *b, uint64_t nb, uint64_t *out) {
    uint64_t i = 0, j = 0, w = 0;
    while (i < na) {
        while (j < nb && b[j] < a[i]) ++j;
        if (j < nb && b[j] == a[i]) { ++i; continue; }
        out[w++] = a[i++];
    }
    return w;
}

/* A U B for sorted unique A, B into out (capacity na+nb).  Returns |out|. */
uint64_t or_union_sorted(const uint64_t *a, uint64_t na, const uint64_t *b, uint64_t nb, uint64_t *out) {
    uint64_t i = 0, j = 0, w = 0;
    while (i < na && j < nb) {
        if (a[i] < b[j]) out[w++] = a[i++];
        else if (b[j] < a[i]) out[w++] = b[j++];
        else { out[w++] = a[i++]; ++j; }
    }
    while (i < na) out[w++] = a[i++];
    while (j < nb) out[w++] = b[j++];
    return w;
}

/* FNV-1a 64 over the little-endian bytes of each packed key in order
 * (offset 0xcbf29ce484222325, prime 0x100000001b3 as in pack.cu:8-9). */
uint64_t or_fnv1a64(const uint64_t *a, uint64_t n) {
    uint64_t h = 0xcbf29ce484222325ULL;
    for (uint64_t i = 0; i < n; ++i) {
        uint64_t k = a[i];
        for (int b = 0; b < 8; ++b) { h ^= (k >> (8 * b)) & 255; h *= 0x100000001b3ULL; }
    }
    return h;
}

/* FNV-1a 64 over a byte string (the published function itself; the key form
 * above is this function over the keys' little-endian bytes). */
uint64_t or_fnv1a64_bytes(const uint8_t *p, uint64_t n) {
    uint64_t h = 0xcbf29ce484222325ULL;
    for (uint64_t i = 0; i < n; ++i) { h ^= p[i]; h *= 0x100000001b3ULL; }
    return h;
}

/* ------------------------------------------------------------------------ */
/* growable u64 vector                                                       */
/* ------------------------------------------------------------------------ */
typedef struct { uint64_t *v; uint64_t n, cap; } vec64;

static int vec_reserve(vec64 *x, uint64_t cap) {
    if (cap <= x->cap) return 0;
    uint64_t c = x->cap ? x->cap : 16;
    while (c < cap) c *= 2;
    uint64_t *p = (uint64_t *)realloc(x->v, c * sizeof(uint64_t));
    if (!p) return -2;
    x->v = p; x->cap = c;
    return 0;
}
static inline int vec_push(vec64 *x, uint64_t k) {
    if (x->n == x->cap && vec_reserve(x, x->n + 1)) return -2;
    x->v[x->n++] = k;
    return 0;
}
static void vec_free(vec64 *x) { free(x->v); x->v = NULL; x->n = x->cap = 0; }

/* ------------------------------------------------------------------------ */
/* join                                                                      */
/* ------------------------------------------------------------------------ */

static inline uint32_t col_of(uint64_t k, int c) { return c ? (uint32_t)k : (uint32_t)(k >> 32); }

/* Inner join of L and R (arity-2 packed tuples) on L.col[lk] == R.col[rk];
 * each output row is the 4-column row L ++ R projected onto out_cols[0..1]
 * (indices into (L.c0, L.c1, R.c0, R.c1)) and packed.  Bag output appended
 * to *out.  R is re-indexed by sorting a (key, other) copy. */
static int join_project(const uint64_t *l, uint64_t nl, const uint64_t *r, uint64_t nr,
                        int lk, int rk, const int out_cols[2], vec64 *out) {
    if (nl == 0 || nr == 0) return 0;
    uint64_t *idx = (uint64_t *)malloc(nr * sizeof(uint64_t));
    if (!idx) return -2;
    for (uint64_t i = 0; i < nr; ++i)  /* (key, other column) */
        idx[i] = ((uint64_t)col_of(r[i], rk) << 32) | col_of(r[i], 1 - rk);
    if (or_sort_u64(idx, nr)) { free(idx); return -2; }
#ifdef _OPENMP
    if (g_threads > 1 && nl >= (1u << 14)) {
        /* two passes over contiguous chunks of L (count, then write at the
         * chunk's offset): the same bag in the same order as below.  The run
         * start of every L row is kept from the first pass. */
        const int T = g_threads;
        uint64_t *off = (uint64_t *)calloc((size_t)T + 1, sizeof(uint64_t));
        uint64_t *lo_of = (uint64_t *)malloc(nl * sizeof(uint64_t));
        uint32_t *cnt_of = (uint32_t *)malloc(nl * sizeof(uint32_t));
        if (!off || !lo_of || !cnt_of) { free(off); free(lo_of); free(cnt_of); free(idx); return -2; }
        #pragma omp parallel num_threads(T)
        {
            const int t = omp_get_thread_num();
            const uint64_t lo = nl * (uint64_t)t / (uint64_t)T, hi = nl * (uint64_t)(t + 1) / (uint64_t)T;
            uint64_t c = 0;
            for (uint64_t i = lo; i < hi; ++i) {
                uint32_t key = col_of(l[i], lk);
                uint64_t a = 0, b = nr;
                while (a < b) { uint64_t m = (a + b) / 2; if ((uint32_t)(idx[m] >> 32) < key) a = m + 1; else b = m; }
                uint64_t e = a;
                while (e < nr && (uint32_t)(idx[e] >> 32) == key) ++e;
                lo_of[i] = a;
                cnt_of[i] = (uint32_t)(e - a);
                c += e - a;
            }
            off[t + 1] = c;
        }
        for (int t = 0; t < T; ++t) off[t + 1] += off[t];
        const uint64_t base = out->n;
        if (vec_reserve(out, base + off[T])) { free(off); free(lo_of); free(cnt_of); free(idx); return -2; }
        #pragma omp parallel num_threads(T)
        {
            const int t = omp_get_thread_num();
            const uint64_t lo = nl * (uint64_t)t / (uint64_t)T, hi = nl * (uint64_t)(t + 1) / (uint64_t)T;
            uint64_t w = base + off[t];
            for (uint64_t i = lo; i < hi; ++i) {
                const uint32_t key = col_of(l[i], lk);
                for (uint64_t j = lo_of[i], e = lo_of[i] + cnt_of[i]; j < e; ++j) {
                    uint32_t row[4];
                    row[0] = (uint32_t)(l[i] >> 32); row[1] = (uint32_t)l[i];
                    row[2 + rk] = key; row[3 - rk] = (uint32_t)idx[j];
                    out->v[w++] = ((uint64_t)row[out_cols[0]] << 32) | row[out_cols[1]];
                }
            }
        }
        free(lo_of);
        free(cnt_of);
        out->n = base + off[T];
        free(off);
        free(idx);
        return 0;
    }
#endif
    for (uint64_t i = 0; i < nl; ++i) {
        uint32_t key = col_of(l[i], lk);
        uint64_t lo = 0, hi = nr;
        while (lo < hi) { uint64_t m = (lo + hi) / 2; if ((uint32_t)(idx[m] >> 32) < key) lo = m + 1; else hi = m; }
        for (uint64_t j = lo; j < nr && (uint32_t)(idx[j] >> 32) == key; ++j) {
            uint32_t row[4];
            row[0] = (uint32_t)(l[i] >> 32); row[1] = (uint32_t)l[i];
            row[2 + rk] = key; row[3 - rk] = (uint32_t)idx[j];
            if (vec_push(out, ((uint64_t)row[out_cols[0]] << 32) | row[out_cols[1]])) { free(idx); return -2; }
        }
    }
    free(idx);
    return 0;
}

/* exported: L join R then project, sorted + deduplicated result */
int64_t or_join_project(const uint64_t *l, uint64_t nl, const uint64_t *r, uint64_t nr,
                        int lk, int rk, int oc0, int oc1, uint64_t **out) {
    vec64 o = {0};
    int oc[2] = {oc0, oc1};
    if (join_project(l, nl, r, nr, lk, rk, oc, &o)) { vec_free(&o); return -2; }
    *out = o.v;
    return (int64_t)o.n;
}
/* exported: size of the inner join bag (no materialisation) */
uint64_t or_join_count(const uint64_t *l, uint64_t nl, const uint64_t *r, uint64_t nr, int lk, int rk) {
    if (!nl || !nr) return 0;
    uint32_t *rkeys = (uint32_t *)malloc(nr * sizeof(uint32_t));
    uint64_t *tmp = (uint64_t *)malloc(nr * sizeof(uint64_t));
    for (uint64_t i = 0; i < nr; ++i) tmp[i] = col_of(r[i], rk);
    or_sort_u64(tmp, nr);
    for (uint64_t i = 0; i < nr; ++i) rkeys[i] = (uint32_t)tmp[i];
    free(tmp);
    uint64_t total = 0;
    for (uint64_t i = 0; i < nl; ++i) {
        uint32_t key = col_of(l[i], lk);
        uint64_t lo = 0, hi = nr;
        while (lo < hi) { uint64_t m = (lo + hi) / 2; if (rkeys[m] < key) lo = m + 1; else hi = m; }
        uint64_t a = lo; hi = nr;
        while (lo < hi) { uint64_t m = (lo + hi) / 2; if (rkeys[m] <= key) lo = m + 1; else hi = m; }
        total += lo - a;
    }
    free(rkeys);
    return total;
}
void or_free(void *p) { free(p); }

/* exported: the row counts of the left-deep two-join body
 *   head(v, o) :- l(v, w), a(w, p), b(p, o)
 * evaluated as (l join a on w) projected to (v, p), then joined with b on p
 * (crates/xlog-logic/src/lower.rs:1795-1850; join output left ++ right,
 * relational.rs:4417-4625).  l, a, b are sorted unique packed (c0 << 32) | c1
 * rows; every id must be below 2^28 (-1 otherwise).  out[0] = the first join's
 * bag, out[1] = its distinct (v, p) pairs, out[2] = the second join's bag over
 * those distinct pairs, out[3] = the second join's bag over the first join's
 * bag.  Counting only: a degree array per relation and, per v (l is sorted by
 * v), a marker array of the p values already seen. */
int or_chain2_counts(const uint64_t *l, uint64_t nl, const uint64_t *a, uint64_t na, const uint64_t *b, uint64_t nb,
                     uint64_t *out) {
    uint32_t mx = 0;
    for (uint64_t i = 0; i < nl; ++i) { mx = mx > (uint32_t)(l[i] >> 32) ? mx : (uint32_t)(l[i] >> 32);
                                        mx = mx > (uint32_t)l[i] ? mx : (uint32_t)l[i]; }
    for (uint64_t i = 0; i < na; ++i) { mx = mx > (uint32_t)(a[i] >> 32) ? mx : (uint32_t)(a[i] >> 32);
                                        mx = mx > (uint32_t)a[i] ? mx : (uint32_t)a[i]; }
    for (uint64_t i = 0; i < nb; ++i) { mx = mx > (uint32_t)(b[i] >> 32) ? mx : (uint32_t)(b[i] >> 32);
                                        mx = mx > (uint32_t)b[i] ? mx : (uint32_t)b[i]; }
    out[0] = out[1] = out[2] = out[3] = 0;
    if (mx >= (1u << 28)) return -1;
    const uint64_t D = (uint64_t)mx + 1;
    uint64_t *a_start = (uint64_t *)calloc(D + 1, sizeof(uint64_t));  /* CSR of a over w */
    uint64_t *deg_b = (uint64_t *)calloc(D, sizeof(uint64_t));
    uint64_t *seen = (uint64_t *)calloc(D, sizeof(uint64_t));         /* 1 + the last v that saw p */
    if (!a_start || !deg_b || !seen) { free(a_start); free(deg_b); free(seen); return -2; }
    for (uint64_t i = 0; i < na; ++i) a_start[(a[i] >> 32) + 1]++;
    for (uint64_t w = 0; w < D; ++w) a_start[w + 1] += a_start[w];
    for (uint64_t i = 0; i < nb; ++i) deg_b[b[i] >> 32]++;
    for (uint64_t i = 0; i < nl; ++i) {
        const uint64_t v = l[i] >> 32, w = (uint32_t)l[i];
        for (uint64_t j = a_start[w]; j < a_start[w + 1]; ++j) {
            const uint32_t pv = (uint32_t)a[j];
            out[0] += 1;
            out[3] += deg_b[pv];
            if (seen[pv] != v + 1) {
                seen[pv] = v + 1;
                out[1] += 1;
                out[2] += deg_b[pv];
            }
        }
    }
    free(a_start);
    free(deg_b);
    free(seen);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* program plans: rules over arity-2 predicates, left-deep bodies           */
/* ------------------------------------------------------------------------ */
/* Layout of the int32 plan array (shared with the GPU library's plan):
 *   [n_rules, then per rule: head_pred, hv0, hv1, n_body, (pred, v0, v1) * n_body]
 * Variables are small non-negative ints.  Bodies are evaluated left-deep in
 * body order, as lowering produces them (crates/xlog-logic/src/lower.rs:1795-1850):
 * the running binding joins the next atom on their shared variable (or, when
 * both of the atom's variables are bound, on both: a cyclic body such as a
 * triangle), and keeps only the variables that a later atom or the head still
 * reads.  A binding holds at most two variables. */

#define MAX_BODY 4
typedef struct { int pred, v[2]; } atom_t;
typedef struct { int head, hv[2], nb; atom_t b[MAX_BODY]; } rule_t;

static int parse_plan(const int32_t *plan, int *nrules, rule_t *rules, int max_rules) {
    int p = 0, nr = plan[p++];
    if (nr < 0 || nr > max_rules) return -1;
    for (int i = 0; i < nr; ++i) {
        rule_t *r = &rules[i];
        r->head = plan[p++]; r->hv[0] = plan[p++]; r->hv[1] = plan[p++]; r->nb = plan[p++];
        if (r->nb < 1 || r->nb > MAX_BODY) return -1;
        for (int j = 0; j < r->nb; ++j) { r->b[j].pred = plan[p++]; r->b[j].v[0] = plan[p++]; r->b[j].v[1] = plan[p++]; }
    }
    *nrules = nr;
    return 0;
}

/* A binding is a bag of packed rows over vars[0..nv) (nv in {1,2}; nv==1
 * stores the value in the low word). */
typedef struct { int nv, vars[2]; vec64 rows; } binding_t;

static int needed_later(const rule_t *r, int from_atom, int var) {
    if (r->hv[0] == var || r->hv[1] == var) return 1;
    for (int j = from_atom; j < r->nb; ++j) if (r->b[j].v[0] == var || r->b[j].v[1] == var) return 1;
    return 0;
}

/* The last join of a body when its two output variables are a binding
 * variable g (not the shared one) and the atom's new variable o: the set
 * { (g, o) : binding (g, s), atom (s, o) } (with the columns of `nxt`'s
 * order) without the bag.  Binding rows are grouped by g; per group the o's of
 * every matching atom row are OR-ed into a bitset over o's domain and the set
 * bits emitted, groups spread over the threads.  idx: the atom relation as
 * sorted (shared << 32) | o.  Returns 1 when it ran, 0 when the domain is too
 * large for per-thread bitsets (the caller then takes the bag path), <0 on
 * OOM. */
static int last_join_grouped(const binding_t *cur, int gpos, const uint64_t *idx, uint64_t nr, int atom_self,
                             int g_first, vec64 *outv) {
    uint32_t maxo = 0;
    for (uint64_t i = 0; i < nr; ++i) if ((uint32_t)idx[i] > maxo) maxo = (uint32_t)idx[i];
    const uint64_t D = (uint64_t)maxo + 1;
    if (D > (1ull << 27)) return 0;
    const uint64_t words = (D + 63) / 64, n = cur->rows.n;
    uint64_t *gp = (uint64_t *)malloc((n ? n : 1) * sizeof(uint64_t));  /* (g << 32) | shared */
    if (!gp) return -2;
    for (uint64_t i = 0; i < n; ++i) {
        const uint64_t row = cur->rows.v[i];
        const uint32_t g = gpos ? (uint32_t)row : (uint32_t)(row >> 32);
        const uint32_t s = gpos ? (uint32_t)(row >> 32) : (uint32_t)row;
        gp[i] = ((uint64_t)g << 32) | s;
    }
    if (or_sort_u64(gp, n)) { free(gp); return -2; }
    /* group starts */
    uint64_t ng = 0;
    uint64_t *gs = (uint64_t *)malloc((n + 1) * sizeof(uint64_t));
    if (!gs) { free(gp); return -2; }
    for (uint64_t i = 0; i < n; ++i)
        if (i == 0 || (gp[i] >> 32) != (gp[i - 1] >> 32)) gs[ng++] = i;
    gs[ng] = n;
    int T = 1;
#ifdef _OPENMP
    T = g_threads > 1 ? g_threads : 1;
#endif
    vec64 *loc = (vec64 *)calloc((size_t)T, sizeof(vec64));
    uint64_t **bits = (uint64_t **)calloc((size_t)T, sizeof(uint64_t *));
    int err = (!loc || !bits);
    for (int t = 0; t < T && !err; ++t)
        if (!(bits[t] = (uint64_t *)calloc(words, sizeof(uint64_t)))) err = 1;
    if (!err) {
#ifdef _OPENMP
        #pragma omp parallel for num_threads(T) schedule(dynamic, 8)
#endif
        for (int64_t q = 0; q < (int64_t)ng; ++q) {
            int t = 0;
#ifdef _OPENMP
            t = omp_get_thread_num();
#endif
            uint64_t *b = bits[t];
            const uint32_t g = (uint32_t)(gp[gs[q]] >> 32);
            uint64_t wlo = words, whi = 0;  /* touched word range */
            for (uint64_t i = gs[q]; i < gs[q + 1]; ++i) {
                const uint32_t key = (uint32_t)gp[i];
                uint64_t lo = 0, hi = nr;
                while (lo < hi) { uint64_t m = (lo + hi) / 2; if ((uint32_t)(idx[m] >> 32) < key) lo = m + 1; else hi = m; }
                for (uint64_t e = lo; e < nr && (uint32_t)(idx[e] >> 32) == key; ++e) {
                    const uint32_t o = (uint32_t)idx[e];
                    if (atom_self && o != key) continue;
                    b[o >> 6] |= 1ull << (o & 63);
                    if ((o >> 6) < wlo) wlo = o >> 6;
                    if ((o >> 6) + 1 > whi) whi = (o >> 6) + 1;
                }
            }
            for (uint64_t w = wlo; w < whi; ++w) {
                uint64_t x = b[w];
                b[w] = 0;
                while (x) {
                    const uint32_t o = (uint32_t)(w * 64 + (uint64_t)__builtin_ctzll(x));
                    x &= x - 1;
                    const uint64_t row = g_first ? (((uint64_t)g << 32) | o) : (((uint64_t)o << 32) | g);
                    if (vec_push(&loc[t], row)) err = 1;
                }
            }
        }
    }
    uint64_t total = 0;
    for (int t = 0; t < T && !err; ++t) total += loc[t].n;
    if (!err && vec_reserve(outv, outv->n + total)) err = 1;
    for (int t = 0; t < T; ++t) {
        if (!err) {
            memcpy(outv->v + outv->n, loc[t].v, loc[t].n * sizeof(uint64_t));
            outv->n += loc[t].n;
        }
        if (loc) vec_free(&loc[t]);
        if (bits) free(bits[t]);
    }
    free(loc);
    free(bits);
    free(gs);
    free(gp);
    return err ? -2 : 1;
}

/* Evaluate one rule body with rel[j] the relation read by atom j.
 * Appends the projected head tuples (bag) to *out. */
static int eval_body(const rule_t *r, const uint64_t *const *rel, const uint64_t *nrel, vec64 *out) {
    /* start from atom 0 */
    binding_t cur = {0};
    {
        const atom_t *a = &r->b[0];
        int keep0 = needed_later(r, 1, a->v[0]), keep1 = needed_later(r, 1, a->v[1]);
        if (a->v[0] == a->v[1]) keep1 = 0;
        cur.nv = 0;
        if (keep0) cur.vars[cur.nv++] = a->v[0];
        if (keep1) cur.vars[cur.nv++] = a->v[1];
        if (vec_reserve(&cur.rows, nrel[0])) return -2;
        for (uint64_t i = 0; i < nrel[0]; ++i) {
            uint64_t k = rel[0][i];
            uint32_t c0 = (uint32_t)(k >> 32), c1 = (uint32_t)k;
            if (a->v[0] == a->v[1] && c0 != c1) continue;
            uint64_t row;
            if (cur.nv == 2) row = k;
            else if (cur.nv == 1) row = keep0 ? c0 : c1;
            else row = 0;
            cur.rows.v[cur.rows.n++] = row;
        }
        if (cur.nv < 2) { cur.rows.n = or_sort_dedup(cur.rows.v, cur.rows.n); }
    }
    for (int j = 1; j < r->nb; ++j) {
        const atom_t *a = &r->b[j];
        /* shared variables between binding and atom */
        int bpos[2], apos[2], ns = 0;
        for (int x = 0; x < cur.nv; ++x)
            for (int y = 0; y < 2; ++y)
                if (cur.vars[x] == a->v[y]) { int dup = 0; for (int z = 0; z < ns; ++z) if (bpos[z] == x) dup = 1; if (!dup) { bpos[ns] = x; apos[ns] = y; ++ns; } }
        if (ns == 2) {
            /* both of the atom's variables are bound: an inner join on two keys
             * (lower.rs compute_join_keys), i.e. the binding rows whose values,
             * in the atom's column order, form a row of the atom */
            const int x0 = apos[0] == 0 ? bpos[0] : bpos[1], x1 = apos[0] == 0 ? bpos[1] : bpos[0];
            uint64_t nr = nrel[j];
            uint64_t *set = (uint64_t *)malloc((nr ? nr : 1) * sizeof(uint64_t));
            if (!set) { vec_free(&cur.rows); return -2; }
            memcpy(set, rel[j], nr * sizeof(uint64_t));
            nr = or_sort_dedup(set, nr);
            binding_t nxt = {0};
            int src[2];
            for (int x = 0; x < cur.nv; ++x)
                if (needed_later(r, j + 1, cur.vars[x])) { nxt.vars[nxt.nv] = cur.vars[x]; src[nxt.nv] = x; nxt.nv++; }
            for (uint64_t i = 0; i < cur.rows.n; ++i) {
                const uint64_t row = cur.rows.v[i];
                const uint32_t bv[2] = {(uint32_t)(row >> 32), (uint32_t)row};
                const uint64_t key = ((uint64_t)bv[x0] << 32) | bv[x1];
                uint64_t lo = 0, hi = nr;
                while (lo < hi) { uint64_t m = (lo + hi) / 2; if (set[m] < key) lo = m + 1; else hi = m; }
                if (lo == nr || set[lo] != key) continue;
                uint64_t o;
                if (nxt.nv == 2) o = ((uint64_t)bv[src[0]] << 32) | bv[src[1]];
                else if (nxt.nv == 1) o = bv[src[0]];
                else o = 0;
                if (vec_push(&nxt.rows, o)) { free(set); vec_free(&cur.rows); vec_free(&nxt.rows); return -2; }
            }
            free(set);
            vec_free(&cur.rows);
            nxt.rows.n = or_sort_dedup(nxt.rows.v, nxt.rows.n);
            cur = nxt;
            continue;
        }
        if (ns != 1) { vec_free(&cur.rows); return -3; }  /* plan shape not supported */
        /* candidate output vars: binding vars ++ atom's non-shared var */
        int allv[3], na = 0;
        for (int x = 0; x < cur.nv; ++x) allv[na++] = cur.vars[x];
        int other = a->v[1 - apos[0]];
        int other_is_new = (other != a->v[apos[0]]);
        for (int x = 0; x < cur.nv; ++x) if (cur.vars[x] == other) other_is_new = 0;
        if (other_is_new) allv[na++] = other;
        binding_t nxt = {0};
        int src[2];
        for (int x = 0; x < na; ++x)
            if (needed_later(r, j + 1, allv[x])) { if (nxt.nv == 2) { vec_free(&cur.rows); return -3; } nxt.vars[nxt.nv] = allv[x]; src[nxt.nv] = x; nxt.nv++; }
        /* index the atom relation by its join column */
        uint64_t nr = nrel[j];
        uint64_t *idx = (uint64_t *)malloc((nr ? nr : 1) * sizeof(uint64_t));
        if (!idx) { vec_free(&cur.rows); return -2; }
        int jk = apos[0];
        for (uint64_t i = 0; i < nr; ++i) idx[i] = ((uint64_t)col_of(rel[j][i], jk) << 32) | col_of(rel[j][i], 1 - jk);
        or_sort_u64(idx, nr);
        int atom_self = (a->v[0] == a->v[1]);
        /* the last join with output (the binding's other variable, the atom's new variable): grouped, no bag */
        if (j == r->nb - 1 && cur.nv == 2 && nxt.nv == 2 && other_is_new) {
            const int gpos = 1 - bpos[0];
            const int gv = cur.vars[gpos];
            if ((nxt.vars[0] == gv && nxt.vars[1] == other) || (nxt.vars[1] == gv && nxt.vars[0] == other)) {
                const int ran = last_join_grouped(&cur, gpos, idx, nr, atom_self, nxt.vars[0] == gv, &nxt.rows);
                if (ran < 0) { free(idx); vec_free(&cur.rows); vec_free(&nxt.rows); return -2; }
                if (ran == 1) {
                    free(idx);
                    vec_free(&cur.rows);
                    nxt.rows.n = or_sort_dedup(nxt.rows.v, nxt.rows.n);
                    cur = nxt;
                    continue;
                }
            }
        }
        /* column of 'other' check when it is an already-bound var (ns would be 2) handled above */
        for (uint64_t i = 0; i < cur.rows.n; ++i) {
            uint64_t row = cur.rows.v[i];
            uint32_t bv[2];
            if (cur.nv == 2) { bv[0] = (uint32_t)(row >> 32); bv[1] = (uint32_t)row; }
            else { bv[0] = (uint32_t)row; bv[1] = 0; }
            uint32_t key = bv[bpos[0]];
            uint64_t lo = 0, hi = nr;
            while (lo < hi) { uint64_t m = (lo + hi) / 2; if ((uint32_t)(idx[m] >> 32) < key) lo = m + 1; else hi = m; }
            for (uint64_t q = lo; q < nr && (uint32_t)(idx[q] >> 32) == key; ++q) {
                uint32_t ov = (uint32_t)idx[q];
                if (atom_self && ov != key) continue;
                uint32_t vals[3] = {bv[0], bv[1], 0};
                if (cur.nv == 1) vals[1] = 0;
                vals[cur.nv] = ov;
                uint64_t o;
                if (nxt.nv == 2) o = ((uint64_t)vals[src[0]] << 32) | vals[src[1]];
                else if (nxt.nv == 1) o = vals[src[0]];
                else o = 0;
                if (vec_push(&nxt.rows, o)) { free(idx); vec_free(&cur.rows); vec_free(&nxt.rows); return -2; }
            }
        }
        free(idx);
        vec_free(&cur.rows);
        /* set semantics: intermediates may be deduplicated */
        nxt.rows.n = or_sort_dedup(nxt.rows.v, nxt.rows.n);
        cur = nxt;
    }
    /* project to the head */
    for (uint64_t i = 0; i < cur.rows.n; ++i) {
        uint64_t row = cur.rows.v[i];
        uint32_t h[2];
        for (int t = 0; t < 2; ++t) {
            int pos = -1;
            for (int x = 0; x < cur.nv; ++x) if (cur.vars[x] == r->hv[t]) pos = x;
            if (pos < 0) { vec_free(&cur.rows); return -3; }
            h[t] = (cur.nv == 2) ? (pos ? (uint32_t)row : (uint32_t)(row >> 32)) : (uint32_t)row;
        }
        if (vec_push(out, ((uint64_t)h[0] << 32) | h[1])) { vec_free(&cur.rows); return -2; }
    }
    vec_free(&cur.rows);
    return 0;
}

/* Semi-naive fixpoint (recursive.rs:447-957).
 *   rel[p], nrel[p]: input relations for every predicate p < n_preds, packed,
 *     any order, duplicates allowed.  IDB predicates (rule heads) start from
 *     their given contents (usually empty).
 *   out_rel[p]: receives a malloc'ed sorted unique array for every IDB pred
 *     (caller frees with or_free); out_n[p] its length.
 *   iterations: loop iterations including the final empty one.
 *   delta_sizes[k]: total |delta| over IDB preds after seed (k=0) and after
 *     loop iteration k (k>=1), up to max_trace entries.
 * Returns 0, -1 bad plan, -2 OOM, -3 unsupported shape, -4 iteration limit. */
int or_seminaive(const int32_t *plan, int n_preds, const uint64_t *const *rel, const uint64_t *nrel,
                 uint64_t max_iterations, uint64_t **out_rel, uint64_t *out_n,
                 uint64_t *iterations, uint64_t *delta_sizes, uint64_t max_trace) {
    rule_t rules[64];
    int nrules;
    if (parse_plan(plan, &nrules, rules, 64)) return -1;
    int is_idb[256] = {0};
    if (n_preds > 256) return -1;
    for (int i = 0; i < nrules; ++i) { if (rules[i].head >= n_preds) return -1; is_idb[rules[i].head] = 1; }
    vec64 full[256], delta[256];
    memset(full, 0, sizeof(full)); memset(delta, 0, sizeof(delta));
    /* EDB relations are read as given; IDB start from their canonical form */
    const uint64_t *R[256]; uint64_t NR[256];
    int rc = 0;
    for (int p = 0; p < n_preds; ++p) {
        if (is_idb[p]) {
            if (vec_reserve(&full[p], nrel[p] + 1)) return -2;
            memcpy(full[p].v, rel[p], nrel[p] * sizeof(uint64_t));
            full[p].n = or_sort_dedup(full[p].v, nrel[p]);
            R[p] = full[p].v; NR[p] = full[p].n;
        } else { R[p] = rel[p]; NR[p] = nrel[p]; }
    }
    /* seed: every rule once against the current store */
    vec64 derived[256];
    memset(derived, 0, sizeof(derived));
    for (int i = 0; i < nrules && !rc; ++i) {
        const uint64_t *ar[MAX_BODY]; uint64_t an[MAX_BODY];
        for (int j = 0; j < rules[i].nb; ++j) { ar[j] = R[rules[i].b[j].pred]; an[j] = NR[rules[i].b[j].pred]; }
        rc = eval_body(&rules[i], ar, an, &derived[rules[i].head]);
    }
    uint64_t seed_delta = 0;
    for (int p = 0; p < n_preds && !rc; ++p) {
        if (!is_idb[p]) continue;
        vec64 *d = &derived[p];
        d->n = or_sort_dedup(d->v, d->n);
        /* delta = full_new \ full_old ; full = full_old U derived */
        vec64 nd = {0}, nf = {0};
        if (vec_reserve(&nd, d->n + 1) || vec_reserve(&nf, d->n + full[p].n + 1)) { rc = -2; break; }
        nd.n = or_diff_sorted(d->v, d->n, full[p].v, full[p].n, nd.v);
        nf.n = or_union_sorted(full[p].v, full[p].n, nd.v, nd.n, nf.v);
        vec_free(&full[p]); vec_free(d);
        full[p] = nf; delta[p] = nd;
        R[p] = full[p].v; NR[p] = full[p].n;
        seed_delta += nd.n;
    }
    if (delta_sizes && max_trace > 0) delta_sizes[0] = seed_delta;
    uint64_t it = 0;
    int converged = 0;
    while (!rc && it < max_iterations) {
        ++it;
        vec64 raw[256];
        memset(raw, 0, sizeof(raw));
        for (int i = 0; i < nrules && !rc; ++i) {
            const rule_t *r = &rules[i];
            /* one variant per recursive scan occurrence with a non-empty delta */
            for (int occ = 0; occ < r->nb && !rc; ++occ) {
                int p = r->b[occ].pred;
                if (!is_idb[p] || delta[p].n == 0) continue;
                const uint64_t *ar[MAX_BODY]; uint64_t an[MAX_BODY];
                for (int j = 0; j < r->nb; ++j) {
                    int q = r->b[j].pred;
                    if (j == occ) { ar[j] = delta[q].v; an[j] = delta[q].n; }
                    else { ar[j] = R[q]; an[j] = NR[q]; }
                }
                rc = eval_body(r, ar, an, &raw[r->head]);
            }
        }
        uint64_t total = 0;
        for (int p = 0; p < n_preds && !rc; ++p) {
            if (!is_idb[p]) continue;
            vec64 *d = &raw[p];
            d->n = or_sort_dedup(d->v, d->n);
            d->n = or_diff_sorted(d->v, d->n, full[p].v, full[p].n, d->v);
            vec_free(&delta[p]);
            delta[p] = *d;
            memset(d, 0, sizeof(*d));
            total += delta[p].n;
        }
        for (int p = 0; p < 256; ++p) vec_free(&raw[p]);
        if (rc) break;
        if (delta_sizes && it < max_trace) delta_sizes[it] = total;
        if (total == 0) { converged = 1; break; }
        for (int p = 0; p < n_preds && !rc; ++p) {
            if (!is_idb[p] || delta[p].n == 0) continue;
            vec64 nf = {0};
            if (vec_reserve(&nf, full[p].n + delta[p].n + 1)) { rc = -2; break; }
            nf.n = or_union_sorted(full[p].v, full[p].n, delta[p].v, delta[p].n, nf.v);
            vec_free(&full[p]);
            full[p] = nf;
            R[p] = full[p].v; NR[p] = full[p].n;
        }
    }
    *iterations = it;
    for (int p = 0; p < n_preds; ++p) {
        vec_free(&delta[p]); vec_free(&derived[p]);
        if (is_idb[p] && !rc) { out_rel[p] = full[p].v; out_n[p] = full[p].n; }
        else { vec_free(&full[p]); if (out_rel) out_rel[p] = NULL; if (out_n) out_n[p] = 0; }
    }
    if (rc) return rc;
    return converged ? 0 : -4;
}

/* Naive fixpoint: R_0 = T(empty) U R_init; R_{k} = R_{k-1} U T(R_{k-1}) until
 * unchanged.  rounds = the k at which R_k == R_{k-1}, which equals the
 * semi-naive iteration count.  Same plan/relation conventions. */
int or_naive(const int32_t *plan, int n_preds, const uint64_t *const *rel, const uint64_t *nrel,
             uint64_t max_rounds, uint64_t **out_rel, uint64_t *out_n, uint64_t *rounds) {
    rule_t rules[64];
    int nrules;
    if (parse_plan(plan, &nrules, rules, 64)) return -1;
    int is_idb[256] = {0};
    for (int i = 0; i < nrules; ++i) is_idb[rules[i].head] = 1;
    vec64 full[256];
    memset(full, 0, sizeof(full));
    const uint64_t *R[256]; uint64_t NR[256];
    for (int p = 0; p < n_preds; ++p) {
        if (is_idb[p]) {
            vec_reserve(&full[p], nrel[p] + 1);
            memcpy(full[p].v, rel[p], nrel[p] * sizeof(uint64_t));
            full[p].n = or_sort_dedup(full[p].v, nrel[p]);
            R[p] = full[p].v; NR[p] = full[p].n;
        } else { R[p] = rel[p]; NR[p] = nrel[p]; }
    }
    int rc = 0;
    uint64_t k = 0;
    int changed = 1;
    for (; !rc && k <= max_rounds; ++k) {
        vec64 t[256];
        memset(t, 0, sizeof(t));
        for (int i = 0; i < nrules && !rc; ++i) {
            const uint64_t *ar[MAX_BODY]; uint64_t an[MAX_BODY];
            for (int j = 0; j < rules[i].nb; ++j) { ar[j] = R[rules[i].b[j].pred]; an[j] = NR[rules[i].b[j].pred]; }
            rc = eval_body(&rules[i], ar, an, &t[rules[i].head]);
        }
        changed = 0;
        for (int p = 0; p < n_preds && !rc; ++p) {
            if (!is_idb[p]) continue;
            t[p].n = or_sort_dedup(t[p].v, t[p].n);
            vec64 nf = {0};
            vec_reserve(&nf, full[p].n + t[p].n + 1);
            nf.n = or_union_sorted(full[p].v, full[p].n, t[p].v, t[p].n, nf.v);
            if (nf.n != full[p].n) changed = 1;
            vec_free(&full[p]);
            full[p] = nf;
            R[p] = full[p].v; NR[p] = full[p].n;
        }
        for (int p = 0; p < 256; ++p) vec_free(&t[p]);
        /* round 0 is the seed; the semi-naive loop counts the rounds after it */
        if (!changed && k > 0) break;
    }
    *rounds = k;
    for (int p = 0; p < n_preds; ++p) {
        if (is_idb[p] && !rc) { out_rel[p] = full[p].v; out_n[p] = full[p].n; }
        else { vec_free(&full[p]); out_rel[p] = NULL; out_n[p] = 0; }
    }
    return rc;
}

/* ------------------------------------------------------------------------ */
/* BFS-layer transitive closure (independent closed form)                    */
/* ------------------------------------------------------------------------ */
/* For every source x, BFS over the edge list.  reach(x, z) holds iff z is at
 * finite distance >= 1 from x.  dist_count[d] += #pairs at shortest distance d
 * (d >= 1, up to max_dist).  Returns the maximum finite distance (the
 * semi-naive iteration count for reach(X,Z) :- reach(X,Y), edge(Y,Z); 1 for an
 * empty edge set, where the loop runs once and finds nothing).
 * If out is non-NULL it receives the sorted closure (capacity n_vertices^2
 * worst case: the caller sizes it from a first call with out == NULL).
 * total receives |closure| and digest its FNV-1a-64. */
int64_t or_bfs_tc(uint32_t n_vertices, const uint32_t *src, const uint32_t *dst, uint64_t m,
                  uint64_t *dist_count, uint64_t max_dist, uint64_t *out, uint64_t *total, uint64_t *digest) {
    uint64_t *deg = (uint64_t *)calloc((size_t)n_vertices + 1, sizeof(uint64_t));
    uint32_t *adj = (uint32_t *)malloc((m ? m : 1) * sizeof(uint32_t));
    int32_t *dist = (int32_t *)malloc((size_t)(n_vertices ? n_vertices : 1) * sizeof(int32_t));
    uint32_t *queue = (uint32_t *)malloc((size_t)(n_vertices ? n_vertices : 1) * sizeof(uint32_t));
    uint64_t *row = (uint64_t *)malloc((size_t)(n_vertices ? n_vertices : 1) * sizeof(uint64_t));
    if (!deg || !adj || !dist || !queue || !row) { free(deg); free(adj); free(dist); free(queue); free(row); return -2; }
    for (uint64_t e = 0; e < m; ++e) deg[src[e] + 1]++;
    for (uint32_t v = 0; v < n_vertices; ++v) deg[v + 1] += deg[v];
    uint64_t *fill = (uint64_t *)malloc(((size_t)n_vertices + 1) * sizeof(uint64_t));
    memcpy(fill, deg, ((size_t)n_vertices + 1) * sizeof(uint64_t));
    for (uint64_t e = 0; e < m; ++e) adj[fill[src[e]]++] = dst[e];
    free(fill);
    int64_t maxd = 0;
    uint64_t tot = 0, h = 0xcbf29ce484222325ULL;
#ifdef _OPENMP
    if (g_threads > 1 && !out && !digest) {
        /* counts only: sources in parallel, each thread with its own BFS state */
        const int T = g_threads;
        uint64_t *dc = dist_count ? (uint64_t *)calloc((size_t)T * max_dist, sizeof(uint64_t)) : NULL;
        #pragma omp parallel num_threads(T) reduction(+ : tot) reduction(max : maxd)
        {
            const int t = omp_get_thread_num();
            int32_t *dl = (int32_t *)malloc((size_t)(n_vertices ? n_vertices : 1) * sizeof(int32_t));
            uint32_t *ql = (uint32_t *)malloc((size_t)(n_vertices ? n_vertices : 1) * sizeof(uint32_t));
            uint64_t *mydc = dc ? dc + (size_t)t * max_dist : NULL;
            for (uint32_t v = 0; v < n_vertices; ++v) dl[v] = -1;
            #pragma omp for schedule(dynamic, 64)
            for (uint32_t x = 0; x < n_vertices; ++x) {
                uint64_t qh = 0, qt = 0;
                for (uint64_t e = deg[x]; e < deg[x + 1]; ++e) {
                    uint32_t z = adj[e];
                    if (dl[z] < 0) { dl[z] = 1; ql[qt++] = z; }
                }
                while (qh < qt) {
                    uint32_t y = ql[qh++];
                    for (uint64_t e = deg[y]; e < deg[y + 1]; ++e) {
                        uint32_t z = adj[e];
                        if (dl[z] < 0) { dl[z] = dl[y] + 1; ql[qt++] = z; }
                    }
                }
                for (uint64_t i = 0; i < qt; ++i) {
                    int32_t dz = dl[ql[i]];
                    if (dz > maxd) maxd = dz;
                    if (mydc && (uint64_t)dz < max_dist) mydc[dz]++;
                    dl[ql[i]] = -1;  /* only the visited vertices are reset */
                }
                tot += qt;
            }
            free(dl); free(ql);
        }
        if (dc) {
            for (int t = 0; t < T; ++t)
                for (uint64_t d = 0; d < max_dist; ++d) dist_count[d] += dc[(size_t)t * max_dist + d];
            free(dc);
        }
        free(deg); free(adj); free(dist); free(queue); free(row);
        if (total) *total = tot;
        return maxd == 0 ? 1 : maxd;
    }
#endif
    for (uint32_t v = 0; v < n_vertices; ++v) dist[v] = -1;
    for (uint32_t x = 0; x < n_vertices; ++x) {
        uint64_t qh = 0, qt = 0, nrow = 0;
        /* x itself is not at distance 0 in the relation: only walks of length >= 1 count */
        for (uint64_t e = deg[x]; e < deg[x + 1]; ++e) {
            uint32_t z = adj[e];
            if (dist[z] < 0) { dist[z] = 1; queue[qt++] = z; }
        }
        while (qh < qt) {
            uint32_t y = queue[qh++];
            for (uint64_t e = deg[y]; e < deg[y + 1]; ++e) {
                uint32_t z = adj[e];
                if (dist[z] < 0) { dist[z] = dist[y] + 1; queue[qt++] = z; }
            }
        }
        /* the row of x in z order: the visited vertices, sorted; then reset them */
        for (uint64_t i = 0; i < qt; ++i) {
            const uint32_t z = queue[i];
            if (dist[z] > maxd) maxd = dist[z];
            if (dist_count && (uint64_t)dist[z] < max_dist) dist_count[dist[z]]++;
            row[nrow++] = ((uint64_t)x << 32) | z;
            dist[z] = -1;
        }
        sort_u64_serial(row, nrow);
        for (uint64_t i = 0; i < nrow; ++i) {
            uint64_t k = row[i];
            for (int b = 0; b < 8; ++b) { h ^= (k >> (8 * b)) & 255; h *= 0x100000001b3ULL; }
        }
        if (out) memcpy(out + tot, row, nrow * sizeof(uint64_t));
        tot += nrow;
    }
    free(deg); free(adj); free(dist); free(queue); free(row);
    if (total) *total = tot;
    if (digest) *digest = h;
    return maxd == 0 ? 1 : maxd;
}
