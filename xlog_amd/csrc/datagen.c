/*
 * Seeded synthetic relation generators for the five workloads of the
 * semi-naive fixpoint path.  Host-only C; the same code feeds the GPU
 * library, the CPU checker and the benchmark, so every consumer sees
 * identical inputs for a given seed.
 *
 * Random source: the LCG of the reference bench generator
 * (crates/xlog-gpu/benches/logic_bench.rs:48-62):
 *     s <- s * 6364136223846793005 + 1   (mod 2^64)
 * The reference reduces the raw state with `% n`.  The low bits of a
 * power-of-two-modulus LCG have period 2^k (bit 0 alternates), so `% n`
 * ties the parity class of consecutive draws together.  Every draw here
 * takes the HIGH 32 bits instead: below(n) = ((s >> 32) * n) >> 32.
 * xlog_gen_ref_random_graph() keeps the reference's exact `% n` form for
 * fidelity with its bench.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>

#define LCG_MUL 6364136223846793005ULL

static inline uint64_t lcg_next(uint64_t *s) {
    *s = *s * LCG_MUL + 1ULL;
    return *s;
}
static inline uint32_t lcg_u32(uint64_t *s) { return (uint32_t)(lcg_next(s) >> 32); }
static inline uint32_t lcg_below(uint64_t *s, uint32_t n) {
    return (uint32_t)(((lcg_next(s) >> 32) * (uint64_t)n) >> 32);
}
/* Uniform in [0, n) for n up to 2^64: 128-bit multiply of a 64-bit draw
 * assembled from two high halves. */
static inline uint64_t lcg_below64(uint64_t *s, uint64_t n) {
    uint64_t hi = lcg_next(s) >> 32, lo = lcg_next(s) >> 32;
    uint64_t r = (hi << 32) | lo;
    return (uint64_t)(((unsigned __int128)r * n) >> 64);
}
static inline double lcg_unit(uint64_t *s) {
    return (double)(lcg_next(s) >> 11) * (1.0 / 9007199254740992.0);
}

uint64_t xlog_gen_lcg_next(uint64_t *state) { return lcg_next(state); }

/* ---- open-addressing set of u64 (stores key+1; 0 = empty) ---------------- */
typedef struct { uint64_t *slot; uint64_t mask; } u64set;

static int u64set_init(u64set *h, uint64_t expect) {
    uint64_t cap = 1024;
    while (cap < 2 * expect + 16) cap <<= 1;
    h->slot = (uint64_t *)calloc(cap, sizeof(uint64_t));
    h->mask = cap - 1;
    return h->slot ? 0 : -1;
}
static void u64set_free(u64set *h) { free(h->slot); h->slot = NULL; }
static inline uint64_t mix64(uint64_t x) {
    x ^= x >> 30; x *= 0xBF58476D1CE4E5B9ULL;
    x ^= x >> 27; x *= 0x94D049BB133111EBULL;
    x ^= x >> 31;
    return x;
}
/* returns 1 if inserted, 0 if already present */
static int u64set_insert(u64set *h, uint64_t key) {
    uint64_t k = key + 1, i = mix64(key) & h->mask;
    for (;;) {
        uint64_t v = h->slot[i];
        if (v == 0) { h->slot[i] = k; return 1; }
        if (v == k) return 0;
        i = (i + 1) & h->mask;
    }
}

/* ---- small deterministic graphs (logic_bench.rs:40-74) ------------------ */

/* 0->1->...->n-1 ; writes n-1 edges */
uint64_t xlog_gen_chain(uint32_t n, uint32_t *src, uint32_t *dst) {
    uint64_t m = n ? (uint64_t)n - 1 : 0;
    for (uint64_t i = 0; i < m; ++i) { src[i] = (uint32_t)i; dst[i] = (uint32_t)i + 1; }
    return m;
}
/* directed cycle 0->1->...->n-1->0 ; writes n edges */
uint64_t xlog_gen_cycle(uint32_t n, uint32_t *src, uint32_t *dst) {
    for (uint32_t i = 0; i < n; ++i) { src[i] = i; dst[i] = (i + 1) % n; }
    return n;
}
/* K_{n,n}: i -> n+j ; writes n*n edges */
uint64_t xlog_gen_complete_bipartite(uint32_t n, uint32_t *src, uint32_t *dst) {
    uint64_t k = 0;
    for (uint32_t i = 0; i < n; ++i)
        for (uint32_t j = 0; j < n; ++j) { src[k] = i; dst[k] = n + j; ++k; }
    return k;
}
/* The reference bench's generator verbatim in behaviour: m draws of
 * (s % n, s % n), duplicates and self-loops kept. */
void xlog_gen_ref_random_graph(uint32_t n, uint64_t m, uint64_t seed, uint32_t *src, uint32_t *dst) {
    uint64_t s = seed;
    for (uint64_t i = 0; i < m; ++i) {
        src[i] = (uint32_t)(lcg_next(&s) % n);
        dst[i] = (uint32_t)(lcg_next(&s) % n);
    }
}

/* ---- configs 1 and 4: G(n, m) digraph, distinct edges, no self-loops ---- */
int xlog_gen_random_digraph(uint32_t n, uint64_t m, uint64_t seed, uint32_t *src, uint32_t *dst) {
    if (n < 2 || (double)m > (double)n * (double)(n - 1)) return -1;
    u64set h;
    if (u64set_init(&h, m)) return -2;
    uint64_t s = seed, k = 0;
    while (k < m) {
        uint32_t a = lcg_below(&s, n), b = lcg_below(&s, n);
        if (a == b) continue;
        if (!u64set_insert(&h, ((uint64_t)a << 32) | b)) continue;
        src[k] = a; dst[k] = b; ++k;
    }
    u64set_free(&h);
    return 0;
}

/* ---- config 2: R(a,b) with Zipf b, S(b,c) with uniform b ---------------- */

/* Bijection on u32 (odd multiplies and xor-shifts), so distinct ranks map to
 * distinct key ids spread over the whole u32 range. */
static inline uint32_t key_of_rank(uint32_t rank, uint32_t salt) {
    uint32_t x = rank ^ salt;
    x *= 0x9E3779B1u; x ^= x >> 15;
    x *= 0x85EBCA77u; x ^= x >> 13;
    x *= 0xC2B2AE3Du; x ^= x >> 16;
    return x;
}
uint32_t xlog_gen_key_of_rank(uint32_t rank, uint64_t seed) {
    return key_of_rank(rank, (uint32_t)(mix64(seed) >> 32));
}

/* Inverse-CDF table for P(k) proportional to (k+1)^-s, k in [0,n). */
static double *powerlaw_cdf(uint32_t n, double s) {
    double *cdf = (double *)malloc((size_t)n * sizeof(double));
    if (!cdf) return NULL;
    double acc = 0.0;
    for (uint32_t k = 0; k < n; ++k) { acc += pow((double)k + 1.0, -s); cdf[k] = acc; }
    return cdf;
}
static inline uint32_t powerlaw_draw(const double *cdf, uint32_t n, uint64_t *st) {
    double u = lcg_unit(st) * cdf[n - 1];
    uint32_t lo = 0, hi = n - 1;             /* first k with cdf[k] > u */
    while (lo < hi) {
        uint32_t mid = lo + (hi - lo) / 2;
        if (cdf[mid] > u) hi = mid; else lo = mid + 1;
    }
    return lo;
}

int xlog_gen_zipf_join(uint64_t n_r, uint64_t n_s, uint32_t n_keys, double zipf_s, uint64_t seed,
                       uint32_t *r_a, uint32_t *r_b, uint32_t *s_b, uint32_t *s_c) {
    if (n_keys == 0) return -1;
    double *cdf = powerlaw_cdf(n_keys, zipf_s);
    if (!cdf) return -2;
    uint32_t salt = (uint32_t)(mix64(seed) >> 32);
    uint64_t s = seed;
    for (uint64_t i = 0; i < n_r; ++i) {
        r_a[i] = lcg_u32(&s);
        r_b[i] = key_of_rank(powerlaw_draw(cdf, n_keys, &s), salt);
    }
    for (uint64_t i = 0; i < n_s; ++i) {
        s_b[i] = key_of_rank(lcg_below(&s, n_keys), salt);
        s_c[i] = lcg_u32(&s);
    }
    free(cdf);
    return 0;
}

/* ---- config 3: packed u64 tuples with injected exact duplicates --------- */

/* Bijective permutation of [0, n) by cycle-walking a bijection of
 * [0, 2^bits) (odd multiply + xor-shift, all mod 2^bits). */
typedef struct { uint64_t mask; unsigned bits; uint64_t k0, k1; } perm_t;
static void perm_init(perm_t *p, uint64_t n, uint64_t seed) {
    unsigned b = 1;
    while (b < 64 && (1ULL << b) < n) ++b;
    p->bits = b; p->mask = (b >= 64) ? ~0ULL : ((1ULL << b) - 1);
    p->k0 = (mix64(seed ^ 0x1111) | 1ULL); p->k1 = (mix64(seed ^ 0x2222) | 1ULL);
}
static inline uint64_t perm_round(const perm_t *p, uint64_t x) {
    unsigned h = p->bits / 2 ? p->bits / 2 : 1;
    x = (x * p->k0) & p->mask; x ^= x >> h;
    x = (x * p->k1) & p->mask; x ^= x >> h;
    x = (x * p->k0) & p->mask;
    return x;
}
static inline uint64_t perm_apply(const perm_t *p, uint64_t x, uint64_t n) {
    do { x = perm_round(p, x); } while (x >= n);
    return x;
}

/* n tuples: F = n - floor(n*dup_num/dup_den) fresh uniform (c0,c1) pairs and
 * D copies of uniformly chosen fresh tuples; tuple j of that sequence is
 * written at position perm(j).  packed = (c0 << 32) | c1. */
int xlog_gen_dup_tuples(uint64_t n, uint32_t dup_num, uint32_t dup_den, uint64_t seed, uint64_t *packed) {
    if (dup_den == 0 || dup_num > dup_den) return -1;
    uint64_t D = (uint64_t)(((unsigned __int128)n * dup_num) / dup_den), F = n - D;
    if (n && F == 0) return -1;
    uint64_t *fresh = (uint64_t *)malloc((size_t)(F ? F : 1) * sizeof(uint64_t));
    if (!fresh) return -2;
    uint64_t s = seed;
    for (uint64_t j = 0; j < F; ++j) {
        uint64_t c0 = lcg_u32(&s), c1 = lcg_u32(&s);
        fresh[j] = (c0 << 32) | c1;
    }
    perm_t p;
    perm_init(&p, n, seed);
    for (uint64_t j = 0; j < F; ++j) packed[perm_apply(&p, j, n)] = fresh[j];
    for (uint64_t j = F; j < n; ++j) packed[perm_apply(&p, j, n)] = fresh[lcg_below64(&s, F)];
    free(fresh);
    return 0;
}

/* ---- config 5: Andersen facts with power-law variable ids --------------- */

/* Fills four relations with n_assign / n_addr / n_load / n_store distinct
 * (v, w) pairs, v != w, both ids drawn from P(k) ~ (k+1)^-alpha over
 * [0, n_vars) and mapped through a seeded Fisher-Yates permutation. */
int xlog_gen_andersen(uint32_t n_vars, double alpha, uint64_t seed,
                      uint64_t n_assign, uint32_t *assign_v, uint32_t *assign_w,
                      uint64_t n_addr, uint32_t *addr_v, uint32_t *addr_o,
                      uint64_t n_load, uint32_t *load_v, uint32_t *load_w,
                      uint64_t n_store, uint32_t *store_v, uint32_t *store_w) {
    if (n_vars < 2) return -1;
    double *cdf = powerlaw_cdf(n_vars, alpha);
    uint32_t *id = (uint32_t *)malloc((size_t)n_vars * sizeof(uint32_t));
    if (!cdf || !id) { free(cdf); free(id); return -2; }
    uint64_t s = seed;
    for (uint32_t i = 0; i < n_vars; ++i) id[i] = i;
    for (uint32_t i = n_vars - 1; i > 0; --i) {
        uint32_t j = lcg_below(&s, i + 1);
        uint32_t t = id[i]; id[i] = id[j]; id[j] = t;
    }
    uint64_t counts[4] = {n_assign, n_addr, n_load, n_store};
    uint32_t *cv[4] = {assign_v, addr_v, load_v, store_v};
    uint32_t *cw[4] = {assign_w, addr_o, load_w, store_w};
    int rc = 0;
    for (int r = 0; r < 4 && rc == 0; ++r) {
        u64set h;
        if (u64set_init(&h, counts[r])) { rc = -2; break; }
        uint64_t k = 0, tries = 0, limit = 64 * counts[r] + 1000000;
        while (k < counts[r]) {
            if (++tries > limit) { rc = -3; break; }
            uint32_t a = id[powerlaw_draw(cdf, n_vars, &s)];
            uint32_t b = id[powerlaw_draw(cdf, n_vars, &s)];
            if (a == b) continue;
            if (!u64set_insert(&h, ((uint64_t)a << 32) | b)) continue;
            cv[r][k] = a; cw[r][k] = b; ++k;
        }
        u64set_free(&h);
    }
    free(cdf); free(id);
    return rc;
}
