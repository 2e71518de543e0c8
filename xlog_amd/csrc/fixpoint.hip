// The semi-naive fixpoint driver of libxlog_hip (Executor::execute_recursive_scc,
// crates/xlog-runtime/src/executor/recursive.rs:447-957): plan parsing, the
// route choice (bitmap chain, hash set, join) and each route's iterations.
// Host code; the operators it calls are in abi.hip (declared in host.hpp),
// the kernels in the other .hip files.
#include "host.hpp"

#include <algorithm>
#include <array>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>

namespace xh {

// ---------------------------------------------------------------------------
// semi-naive fixpoint driver (Executor::execute_recursive_scc,
// crates/xlog-runtime/src/executor/recursive.rs:447-957)
// ---------------------------------------------------------------------------
namespace {

constexpr int MAX_BODY = 4;
struct Atom { int pred, v[2]; };
// delta_at >= 0: a variant of a rule (its body reordered to start at the
// atom that reads the delta): the host loop evaluates only that variant
struct Rule { int head, hv[2], nb; Atom b[MAX_BODY]; int delta_at = -1; };

std::vector<Rule> parse_plan(const int32_t *plan, uint32_t n_preds) {
    XH_REQUIRE(plan, XLOG_HIP_INVALID_ARG, "plan is NULL");
    int p = 0, nr = plan[p++];
    XH_REQUIRE(nr >= 0 && nr <= 256, XLOG_HIP_INVALID_ARG, "plan: bad rule count");
    std::vector<Rule> rules(nr);
    for (int i = 0; i < nr; ++i) {
        Rule &r = rules[i];
        r.head = plan[p++]; r.hv[0] = plan[p++]; r.hv[1] = plan[p++]; r.nb = plan[p++];
        XH_REQUIRE(r.head >= 0 && (uint32_t)r.head < n_preds, XLOG_HIP_INVALID_ARG, "plan: head predicate out of range");
        XH_REQUIRE(r.nb >= 1 && r.nb <= MAX_BODY, XLOG_HIP_INVALID_ARG, "plan: body must have 1..4 atoms");
        for (int j = 0; j < r.nb; ++j) {
            r.b[j].pred = plan[p++]; r.b[j].v[0] = plan[p++]; r.b[j].v[1] = plan[p++];
            XH_REQUIRE(r.b[j].pred >= 0 && (uint32_t)r.b[j].pred < n_preds, XLOG_HIP_INVALID_ARG,
                       "plan: body predicate out of range");
        }
    }
    return rules;
}

bool needed_later(const Rule &r, int from, int var) {
    if (r.hv[0] == var || r.hv[1] == var) return true;
    for (int j = from; j < r.nb; ++j)
        if (r.b[j].v[0] == var || r.b[j].v[1] == var) return true;
    return false;
}

// The join steps of a rule body, left-deep in body order (each atom after
// the first shares one variable with the running binding, which keeps the two
// variables a later atom or the head reads).  Step j >= 1 joins binding
// column bpos with column apos of atom j and keeps candidate values sel[0],
// sel[1] of (binding 0, binding 1, shared, atom's other); a one-atom body
// projects its columns head[0], head[1].  An atom whose two variables are
// both bound (a cyclic body: the reference's left-deep lowering joins it on
// both keys, lower.rs build_join_tree / compute_join_keys) is a filter step:
// the binding rows whose values, in the atom's column order, form a row of
// the atom (binding column bpos holds the atom's first column); sel then
// picks among the binding's two values.
struct JoinPlanStep {
    int bpos = 0, apos = 0, sel[2] = {0, 0};
    bool filter = false;
};
struct BodyPlan {
    JoinPlanStep step[MAX_BODY];
    int head[2] = {0, 1};
    // the body's output keeps the first atom's first column as its high word
    // (each step keeps binding value 0 first): read from a sorted relation,
    // it comes out grouped by that column, in ascending order
    bool grouped = false;
};
BodyPlan plan_body(const Rule &r) {
    BodyPlan bp;
    const Atom &a0 = r.b[0];
    XH_REQUIRE(a0.v[0] != a0.v[1], XLOG_HIP_UNSUPPORTED, "plan: repeated variable inside an atom");
    bool k0 = needed_later(r, 1, a0.v[0]), k1 = needed_later(r, 1, a0.v[1]);
    XH_REQUIRE(k0 && k1, XLOG_HIP_UNSUPPORTED, "plan: first atom must bind two live variables");
    int vars[2] = {a0.v[0], a0.v[1]};
    if (r.nb == 1) {
        int h0 = (r.hv[0] == vars[0]) ? 0 : (r.hv[0] == vars[1] ? 1 : -1);
        int h1 = (r.hv[1] == vars[0]) ? 0 : (r.hv[1] == vars[1] ? 1 : -1);
        XH_REQUIRE(h0 >= 0 && h1 >= 0, XLOG_HIP_UNSUPPORTED, "plan: head variable not bound by the body");
        bp.head[0] = h0;
        bp.head[1] = h1;
        bp.grouped = h0 == 0;
        return bp;
    }
    bp.grouped = true;
    for (int j = 1; j < r.nb; ++j) {
        const Atom &a = r.b[j];
        XH_REQUIRE(a.v[0] != a.v[1], XLOG_HIP_UNSUPPORTED, "plan: repeated variable inside an atom");
        int bpos = -1, apos = -1, nshared = 0;
        for (int x = 0; x < 2; ++x)
            for (int y = 0; y < 2; ++y)
                if (vars[x] == a.v[y]) { bpos = x; apos = y; ++nshared; }
        XH_REQUIRE(nshared == 1 || nshared == 2, XLOG_HIP_UNSUPPORTED,
                   "plan: each atom must share a variable with the atoms before it");
        if (nshared == 2) {
            JoinPlanStep &st = bp.step[j];
            st.filter = true;
            st.apos = 0;  // probed through the atom's index on its first column
            st.bpos = vars[0] == a.v[0] ? 0 : 1;
            st.sel[0] = 0;
            st.sel[1] = 1;
            if (j == r.nb - 1)
                for (int t = 0; t < 2; ++t) {
                    const int f = vars[0] == r.hv[t] ? 0 : (vars[1] == r.hv[t] ? 1 : -1);
                    XH_REQUIRE(f >= 0, XLOG_HIP_UNSUPPORTED, "plan: head variable not bound by the body");
                    st.sel[t] = f;
                }
            bp.grouped = bp.grouped && st.sel[0] == 0;
            const int v0 = vars[st.sel[0]], v1 = vars[st.sel[1]];
            vars[0] = v0;
            vars[1] = v1;
            continue;
        }
        int other = a.v[1 - apos];
        // candidate values: v0 = binding var 0, v1 = binding var 1, v2 = shared, v3 = other
        int cand_var[4] = {vars[0], vars[1], a.v[apos], other};
        int sel[2], ns = 0;
        if (j == r.nb - 1) {
            for (int t = 0; t < 2; ++t) {
                int f = -1;
                for (int c = 0; c < 4; ++c) if (cand_var[c] == r.hv[t]) { f = c; break; }
                XH_REQUIRE(f >= 0, XLOG_HIP_UNSUPPORTED, "plan: head variable not bound by the body");
                sel[ns++] = f;
            }
        } else {
            int seen[4] = {-1, -1, -1, -1}, nseen = 0;
            for (int c = 0; c < 4; ++c) {
                int v = cand_var[c];
                bool dup = false;
                for (int q = 0; q < nseen; ++q) if (seen[q] == v) dup = true;
                if (dup) continue;
                seen[nseen++] = v;
                if (needed_later(r, j + 1, v)) {
                    XH_REQUIRE(ns < 2, XLOG_HIP_UNSUPPORTED, "plan: more than two live variables");
                    sel[ns++] = c;
                }
            }
            XH_REQUIRE(ns == 2, XLOG_HIP_UNSUPPORTED, "plan: intermediate binding must keep two variables");
        }
        bp.step[j].bpos = bpos;
        bp.step[j].apos = apos;
        bp.step[j].sel[0] = sel[0];
        bp.step[j].sel[1] = sel[1];
        bp.grouped = bp.grouped && sel[0] == 0;
        vars[0] = cand_var[sel[0]];
        vars[1] = cand_var[sel[1]];
    }
    return bp;
}

// Scalars of a queue of iterations (Driver::run_queue) live in one device
// array that is read back at once; word 0 holds the stop flag (0, or the
// queue position + 1 of the first iteration that could not run within its
// bounds).  These single-thread kernels check a count against its bound and
// keep the sums the next launches read.
// After a join step's count: the step's rows must fit its bound (with the
// rows emitted before it into the same candidate buffer: base_in) and the
// join-row limit; the count is kept in slot and the next emit's base in
// base_out.  Runs before the emit, which writes at *base_in.
struct QStep {
    const uint64_t *tot;
    const uint64_t *base_in;
    uint64_t *base_out;
    uint64_t *slot;
    uint64_t cap, limit;
};
__global__ void k_q_step(QStep a, uint32_t *stop, uint32_t code) {
    if (*stop) return;
    const uint64_t t = *a.tot, b = a.base_in ? *a.base_in : 0ull;
    if (b + t > a.cap || (a.limit && t > a.limit)) {
        *a.slot = t;  // the count that did not fit: the host sizes the next queue with it
        atomicCAS(stop, 0u, code);
        return;
    }
    *a.slot = t;
    if (a.base_out) *a.base_out = b + t;
}
// A filtered join step (its outputs appended at *taken): before the emit, the
// bag within the join-row limit and the count before it; after, its outputs
// (the count's growth) in its slot, and the count within the buffer.
struct QFilt {
    const uint64_t *bag;
    uint64_t *taken, *before, *slot;
    uint64_t limit, cap;
};
__global__ void k_q_fstart(QFilt a, uint32_t *stop, uint32_t code) {
    if (*stop) return;
    const uint64_t t = *a.bag;
    if (a.limit && t > a.limit) {
        *a.slot = t;
        atomicCAS(stop, 0u, code);
        return;
    }
    *a.before = *a.taken;
}
__global__ void k_q_fend(QFilt a, uint32_t *stop, uint32_t code) {
    if (*stop) return;
    const uint64_t t = *a.taken;
    *a.slot = t - *a.before;
    if (t > a.cap) atomicCAS(stop, 0u, code);
}
// After the set differences, before the merges: the iteration's delta total,
// and every head's R after the merge, which must fit its bound.
constexpr uint32_t QMAX_HEADS = 16;
struct QEnd {
    const uint64_t *nD, *pR;
    uint64_t *nR, *total;
    uint32_t heads;
    uint64_t rcap[QMAX_HEADS];
};
__global__ void k_q_end(QEnd a, uint32_t *stop, uint32_t code) {
    if (*stop) return;
    uint64_t t = 0;
    for (uint32_t h = 0; h < a.heads; ++h) {
        t += a.nD[h];
        if (a.pR[h] + a.nD[h] > a.rcap[h]) {
            atomicCAS(stop, 0u, code);
            return;
        }
    }
    *a.total = t;
    for (uint32_t h = 0; h < a.heads; ++h) a.nR[h] = a.pR[h] + a.nD[h];
}

// The rows of a queued iteration's index over an IDB relation read in full:
// the base run's (known on the host) and the recent run's (on the device, at
// most its bound).
// A count that must not pass its bound (a buffer written up to the bound):
// past it, the queue stops at this iteration.
__global__ void k_q_cap(const uint64_t *d_n, uint64_t bound, uint32_t *stop, uint32_t code) {
    if (*stop) return;
    if (*d_n > bound) atomicCAS(stop, 0u, code);
}
__global__ void k_q_rows(uint64_t *out, uint64_t base, const uint64_t *d_recent, uint64_t recent_bound,
                         const uint32_t *stop) {
    if (*stop) return;
    const uint64_t r = *d_recent;
    *out = base + (r < recent_bound ? r : recent_bound);
}

// Queued hash-route steps: any of the overflow flags of the steps before
// this one (which then do nothing) as a stop word, and a relation's rows after
// a step (its rows before it, on the device, plus the step's appends, at most
// their bound).
__global__ void k_any_set(const unsigned long long *flags, uint32_t n, uint32_t *out) {
    uint32_t a = 0;
    for (uint32_t i = 0; i < n; ++i) a |= flags[i] != 0ull ? 1u : 0u;
    *out = a;
}
__global__ void k_add_rows(uint64_t *out, const uint64_t *d_a, const uint64_t *d_b, uint64_t b_bound,
                           const uint32_t *stop) {
    if (*stop) return;
    const uint64_t b = *d_b;
    *out = *d_a + (b < b_bound ? b : b_bound);
}

// device-resident canonical packed relation
struct DRel {
    uint64_t *k = nullptr;
    uint64_t n = 0;
    bool owned = false;
    uint64_t version = 0;
};

struct Driver {
    Ctx *ctx;
    std::vector<Rule> rules;
    uint32_t n_preds;
    std::vector<bool> idb;
    std::vector<DRel> full, delta;
    uint64_t version_counter = 1;
    uint64_t max_join_rows = 0;  // 0: no limit on a body join's bag size
    uint64_t cur_iter = 0;       // the loop iteration in progress (the reference's counter, recursive.rs:619-620)
    uint32_t digits = 0;         // varying digits of packed tuples over the value domain (0: from the histograms)
    uint64_t domain = 0;         // largest input id + 1: every derived value is an input value (0: unknown)
    // join-index cache keyed by (relation buffer, column, version)
    struct CacheKey {
        const uint64_t *k; int col; uint64_t version;
        bool operator<(const CacheKey &o) const {
            return std::tie(k, col, version) < std::tie(o.k, o.col, o.version);
        }
    };
    std::map<CacheKey, std::unique_ptr<JoinIndex>> cache;

    // The queued join route keeps R in two sorted runs: full[p] (the base run)
    // and small[p], the recent run every delta is merged into (see run_queue).
    std::vector<DRel> small;
    bool q_learned = false;  // the last queue stopped and its counts changed the bounds' inputs
    // R of a head as a bit matrix (domain rows of ceil(domain / 64) u64 words) for the queue's group
    // bitmaps: m[cur] holds R as it stood when full[p] and small[p] had versions vfull and vsmall, or,
    // with `lags`, R of `rows` rows while full[p] and small[p] still hold R as it was then (a queue that
    // kept R only in the matrix adds its rows there; bitr_settle writes them back); m[cur ^ 1] is the
    // queue's working copy
    struct BitR {
        Buf<uint64_t> m[2];
        int cur = 0;
        uint64_t vfull = 0, vsmall = 0, domain = 0, rows = 0;
        bool valid = false, lags = false;
    };
    std::vector<BitR> bitr;
    bool bitr_current(uint32_t p) const {
        return p < bitr.size() && bitr[p].valid && bitr[p].vfull == full[p].version &&
               bitr[p].vsmall == small[p].version;
    }
    void bitr_stamp(uint32_t p) {
        bitr[p].valid = true;
        bitr[p].vfull = full[p].version;
        bitr[p].vsmall = small[p].version;
    }
    // R's rows, and those past the base run (the recent run's, or what the matrix holds past the base run)
    uint64_t r_rows(int p) const {
        return (size_t)p < bitr.size() && bitr[p].lags ? bitr[p].rows : full[p].n + small[p].n;
    }
    uint64_t recent_rows(int p) const { return r_rows(p) - full[p].n; }
    // R's runs brought up to the matrix: R emitted from it in order as one base run
    void bitr_settle(uint32_t p) {
        if (p >= bitr.size() || !bitr[p].lags) return;
        BitR &b = bitr[p];
        DRel r;
        r.n = bitmap_emit(ctx, b.m[b.cur].p, (uint32_t)b.domain, (b.domain + 63) / 64, &r.k, XLOG_HIP_KERNEL_MERGE,
                          b.rows);
        r.owned = r.k != nullptr;
        r.version = version_counter++;
        release(full[p]);
        release(small[p]);
        full[p] = r;
        b.lags = false;
        bitr_stamp(p);
    }
    void bitr_settle_all() {
        for (uint32_t p = 0; p < bitr.size(); ++p) bitr_settle(p);
    }

    ~Driver() {
        cache.clear();
        for (auto &r : full) if (r.owned) ctx->free(r.k);
        for (auto &r : delta) if (r.owned) ctx->free(r.k);
        for (auto &r : small) if (r.owned) ctx->free(r.k);
    }
    // R of p in one run again: the recent run merged into the base run
    void compact(uint32_t p) {
        if (p >= small.size()) return;
        const bool bits = bitr_current(p);
        if (small[p].n) {
            DRel m = merge(full[p], small[p]);
            release(full[p]);
            full[p] = m;
        }
        release(small[p]);
        if (bits) bitr_stamp(p);  // the same rows
    }
    void compact_all() {
        for (uint32_t p = 0; p < small.size(); ++p) compact(p);
    }

    const JoinIndex &index_of(const DRel &rel, int col) {
        CacheKey key{rel.k, col, rel.version};
        auto it = cache.find(key);
        if (it != cache.end()) return *it->second;
        std::unique_ptr<JoinIndex> J(new JoinIndex());
        build_join_index(ctx, rel.k, rel.n, 2, col, true, *J);
        auto &ref = *J;
        cache[key] = std::move(J);
        return ref;
    }
    // An index whose payloads ascend inside each run: index_of's on the first
    // column (the rows are sorted), a second-column index with its payloads
    // sorted otherwise (cached apart from index_of's)
    const JoinIndex &sorted_index_of(const DRel &rel, int col) {
        if (col == 0) return index_of(rel, 0);
        CacheKey key{rel.k, 2 + col, rel.version};
        auto it = cache.find(key);
        if (it != cache.end()) return *it->second;
        std::unique_ptr<JoinIndex> J(new JoinIndex());
        build_join_index(ctx, rel.k, rel.n, 2, col, true, *J, true);
        auto &ref = *J;
        cache[key] = std::move(J);
        return ref;
    }
    void drop_index(const DRel &rel) {
        for (auto it = cache.begin(); it != cache.end();)
            if (it->first.k == rel.k) it = cache.erase(it); else ++it;
    }

    // An index over an IDB relation whose rows are on the device (a queued
    // iteration's R): rows r[0, cnt[0]) sorted, cnt[0] at most the bound the
    // buffers are sized for, indexed on column col (the second through a sorted
    // copy of the rows with their words exchanged): runs, a table for at most
    // min(bound, domain) runs (every value is below the domain) and payloads,
    // rebuilt with device counts and no read-back.
    struct DevIndex {
        int pred = 0, col = 0;
        JoinIndex J;
        Owned srt, alt;
        Buf<uint32_t> run_key;
        Buf<uint64_t> run_start, cnt;  // cnt[0]: the rows (written by the caller), cnt[1]: the runs
        uint64_t runs_bound = 0;
        explicit DevIndex(Ctx *c) : srt(c), alt(c) {}
    };
    void dev_index_alloc(DevIndex &d, uint64_t bound) {
        const uint64_t nr = std::max<uint64_t>(bound, 1);
        d.runs_bound = std::min(nr, domain ? domain : nr);
        if (d.col) {
            d.srt.reset(alloc_keys(ctx, nr));
            d.alt.reset(alloc_keys(ctx, nr));
        }
        d.run_key = Buf<uint32_t>(ctx, nr);
        d.run_start = Buf<uint64_t>(ctx, nr + 1);
        d.cnt = Buf<uint64_t>(ctx, 2);
        fill_u64(ctx, d.cnt.p, 0ull, 2);
        uint64_t slots = 1024;
        while (slots < 2 * d.runs_bound) slots <<= 1;
        d.J.ix.table = Buf<unsigned long long>(ctx, 2 * slots);
        d.J.ix.table_mask = slots - 1;
        d.J.ix.nruns = d.runs_bound;
        d.J.payload = Buf<uint32_t>(ctx, nr);
        d.J.n = nr;
    }
    // r holds at least nr (<= the allocated bound) rows' room; a raised stop skips the work
    void dev_index_build(DevIndex &d, const uint64_t *r, uint64_t nr, const uint32_t *stop) {
        if (nr == 0) {  // no rows yet: an empty table (cnt[1] is still 0)
            run_index_insert_dev(ctx, d.run_key.p, d.run_start.p, d.cnt.p + 1, 0, d.cnt.p, d.J.ix, stop);
            return;
        }
        const uint64_t *sk = r;
        if (d.col) {
            swap_words(ctx, r, nr, d.srt.p);  // over the bound: the rows past the count are not sorted
            uint64_t *ka = d.srt.p, *kb = d.alt.p;
            radix_sort_dev(ctx, &ka, &kb, nr, d.cnt.p, digits, stop);
            sk = ka;
        }
        select_runs(ctx, sk, nr, d.run_key.p, d.run_start.p, d.cnt.p + 1, d.cnt.p);
        run_index_insert_dev(ctx, d.run_key.p, d.run_start.p, d.cnt.p + 1, d.runs_bound, d.cnt.p, d.J.ix, stop);
        low_words(ctx, sk, nr, d.J.payload.p);
    }

    // Evaluate a rule body; rel[j] is the relation atom j reads.  Appends the
    // head tuples (bag, packed) to `out` as owned device buffers.
    // Rows in and out of every join step of every rule body, from the last
    // evaluation that ran it: the queued iterations size their bounds from
    // these ratios.  obs[ri][j] = {left rows, output rows} of step j >= 1.
    std::vector<std::array<std::pair<uint64_t, uint64_t>, MAX_BODY>> obs;
    // per predicate: the share of its candidates that were new in its last
    // iteration with candidates (the queued iterations' delta estimate), and
    // its last two delta sizes (their ratio predicts the end of a decay)
    std::vector<double> nov;
    std::vector<std::array<uint64_t, 2>> dlast;
    void note_delta(uint32_t p, uint64_t n) { dlast[p] = {dlast[p][1], n}; }

    // A triangle-shaped body: three atoms over three variables, every pair of
    // variables in one atom, the head two of them (u, v).  M is the atom over
    // (u, v), P the one over (u, w), Q the one over (w, v), where w is the
    // variable the head drops.  Its tuples are the rows (u, v) of M for which
    // some w is in both u's run of P and v's run of Q: a worst-case-optimal
    // (generic-join) evaluation, variable order u, v, w, that never writes the
    // pairs of the left-deep plan's first join (the reference promotes such
    // bodies to Free Join, promote.rs:1590-1640; its binary fallback is the
    // left-deep plan, whose result is the same set).
    struct Triangle {
        int m = -1, p = -1, q = -1;
        int mask_swap = 0;  // M's rows are (v, u)
        int pcol = 0, qcol = 0;  // the column of u in P and of v in Q
    };
    static bool triangle_shape(const Rule &r, Triangle &t) {
        if (r.nb != 3 || r.hv[0] == r.hv[1]) return false;
        int vs[6], nv = 0;
        for (int j = 0; j < 3; ++j) {
            if (r.b[j].v[0] == r.b[j].v[1]) return false;
            for (int c = 0; c < 2; ++c) {
                bool seen = false;
                for (int k = 0; k < nv; ++k) seen = seen || vs[k] == r.b[j].v[c];
                if (!seen) vs[nv++] = r.b[j].v[c];
            }
        }
        if (nv != 3) return false;
        const int u = r.hv[0], v = r.hv[1];
        int w = -1;
        bool hu = false, hvv = false;
        for (int k = 0; k < 3; ++k) {
            if (vs[k] == u) hu = true;
            else if (vs[k] == v) hvv = true;
            else w = vs[k];
        }
        if (!hu || !hvv || w < 0) return false;
        auto over = [](const Atom &a, int x, int y) {
            return (a.v[0] == x && a.v[1] == y) || (a.v[0] == y && a.v[1] == x);
        };
        for (int j = 0; j < 3; ++j) {
            if (over(r.b[j], u, v)) t.m = j;
            else if (over(r.b[j], u, w)) t.p = j;
            else if (over(r.b[j], w, v)) t.q = j;
        }
        if (t.m < 0 || t.p < 0 || t.q < 0) return false;
        t.mask_swap = r.b[t.m].v[0] != u;
        t.pcol = r.b[t.p].v[0] == u ? 0 : 1;
        t.qcol = r.b[t.q].v[0] == v ? 0 : 1;
        return true;
    }
    // The generic join when it reads less than the left-deep plan's first join
    // writes: M's rows (each a lookup and an intersection) against the rows of
    // atom 0 times the average run of atom 1 on their shared column.
    // XLOG_HIP_WCOJ=1 / =0 takes it always / never.
    bool use_triangle(const Rule &r, const DRel *const *rel, const Triangle &t) {
        const char *e = getenv("XLOG_HIP_WCOJ");
        if (e && e[0] == '0') return false;
        if (e && e[0] == '1') return true;
        if (rel[0]->n == 0 || rel[1]->n == 0 || rel[t.m]->n == 0) return false;
        int apos = -1;
        for (int x = 0; x < 2 && apos < 0; ++x)
            for (int y = 0; y < 2; ++y)
                if (r.b[0].v[x] == r.b[1].v[y]) apos = y;
        if (apos < 0) return false;
        const JoinIndex &J = index_of(*rel[1], apos);
        const double run = J.ix.nruns ? (double)J.n / (double)J.ix.nruns : 0.0;
        return (double)rel[0]->n * run > 4.0 * (double)rel[t.m]->n;
    }
    void eval_triangle(const DRel *const *rel, const Triangle &t, Bags &out) {
        const DRel &M = *rel[t.m], &P = *rel[t.p], &Q = *rel[t.q];
        if (M.n == 0 || P.n == 0 || Q.n == 0) return;
        const JoinIndex &JP = sorted_index_of(P, t.pcol);
        const JoinIndex &JQ = sorted_index_of(Q, t.qcol);
        Buf<uint8_t> flags(ctx, M.n);
        wcoj_triangle_flags(ctx, M.k, M.n, t.mask_swap, JP.ix, JP.payload.p, JQ.ix, JQ.payload.p, flags.p);
        Owned kept(ctx, alloc_keys(ctx, M.n));
        Buf<uint64_t> cnt(ctx, 1);
        select_flags(ctx, M.k, flags.p, M.n, kept.p, cnt.p);
        ctx->read_scalars(cnt.p, 1);
        const uint64_t n = ctx->host_scalars[0];
        if (n == 0) return;
        if (t.mask_swap) {  // the head's order, (u, v)
            Owned o(ctx, alloc_keys(ctx, n));
            swap_words(ctx, kept.p, n, o.p);
            kept.reset(o.release());
        }
        out.add(kept, n, 0);
    }

    // ri >= 0: record the join steps' sizes in obs[ri]
    void eval_body(const Rule &r, const DRel *const *rel, Bags &out, ProbeJob *pre, int ri = -1) {
        Triangle tri;
        if (triangle_shape(r, tri)) {
            // a triangle whose left-deep plan would keep three variables has only this evaluation
            bool left_deep = true;
            try {
                (void)plan_body(r);
            } catch (const Error &) {
                left_deep = false;
            }
            const char *e = getenv("XLOG_HIP_WCOJ");
            if (!(e && e[0] == '0') && (!left_deep || use_triangle(r, rel, tri))) {
                eval_triangle(rel, tri, out);
                return;
            }
        }
        const BodyPlan bp = plan_body(r);
        const uint64_t *bk = rel[0]->k;
        uint64_t bn = rel[0]->n;
        Owned owned(ctx);  // the binding when an earlier join of this body made it
        if (bn == 0) return;
        const uint64_t src_rows = bn;
        if (r.nb == 1) {
            // head projection of a single atom
            const int h0 = bp.head[0], h1 = bp.head[1];
            Owned go(ctx, static_cast<uint64_t *>(ctx->alloc(bn * sizeof(uint64_t))));
            uint64_t *o = go.p;
            if (h0 == 0 && h1 == 1) copy_d2d(ctx, o, bk, bn);
            else if (h0 == 1 && h1 == 0) swap_words(ctx, bk, bn, o);
            else {
                project_pairs(ctx, bk, bn, h0, h1, o);
            }
            out.add(go, bn, bp.grouped ? group_bound(bn) : 0);
            return;
        }
        for (int j = 1; j < r.nb; ++j) {
            const JoinPlanStep &st = bp.step[j];
            const DRel &ar = *rel[j];
            uint64_t *o = nullptr;
            uint64_t on = 0;
            if (ar.n != 0 && st.filter) {
                on = filter_step(bk, bn, st, index_of(ar, 0), &o);
            } else if (ar.n != 0) {
                int oc[4] = {st.sel[0], st.sel[1], 0, 0};
                if (j == 1 && pre) {  // the count pass ran with the delta's count still on the device
                    on = join_emit(ctx, *pre, oc, &o, max_join_rows, digits);
                } else {
                    const JoinIndex &J = index_of(ar, st.apos);
                    on = join_step(ctx, bk, bn, st.bpos, J, oc, &o, max_join_rows, digits);
                }
            }
            if (ri >= 0 && ri < (int)obs.size()) obs[ri][j] = {bn, on};
            owned.reset(o);
            bk = o;
            bn = on;
            if (bn == 0) return;
        }
        out.add(owned, bn, bp.grouped ? group_bound(src_rows) : 0);
    }

    // A filter step (plan_body): the rows of the binding bk whose values, in
    // the atom's column order, are a row of the atom (J: its index on the
    // first column, whose payloads ascend inside each run), in their order,
    // then the binding's two values as sel picks them.
    uint64_t filter_step(const uint64_t *bk, uint64_t bn, const JoinPlanStep &st, const JoinIndex &J, uint64_t **out) {
        Buf<uint8_t> flags(ctx, bn);
        join_match2_flags(ctx, bk, bn, st.bpos, J.ix, J.payload.p, flags.p);
        Owned kept(ctx, alloc_keys(ctx, bn));
        Buf<uint64_t> cnt(ctx, 1);
        select_flags(ctx, bk, flags.p, bn, kept.p, cnt.p);
        ctx->read_scalars(cnt.p, 1);
        const uint64_t n = ctx->host_scalars[0];
        if (n && !(st.sel[0] == 0 && st.sel[1] == 1)) {
            Owned o(ctx, alloc_keys(ctx, n));
            if (st.sel[0] == 1 && st.sel[1] == 0) {
                swap_words(ctx, kept.p, n, o.p);
            } else {
                project_pairs(ctx, kept.p, n, st.sel[0], st.sel[1], o.p);
            }
            kept.reset(o.release());
        }
        *out = n ? kept.release() : nullptr;
        return n;
    }

    // Groups of a body's output that keeps the high word of `rows` sorted
    // source rows: at most one per row and one per value of the domain.
    uint64_t group_bound(uint64_t rows) const {
        return std::max<uint64_t>(1, domain ? std::min(rows, domain) : rows);
    }
    // A grouped bag whose groups average at most this many rows is sorted by
    // one short-run pass (runs of more than 256 rows fall back to the digit
    // passes); with longer groups the digit passes run directly.
    static constexpr uint64_t SHORT_GROUP_ROWS = 64;

    // concat bags, sort, unique, minus full -> new canonical delta.  The count
    // stays on the device (cnt); d.n is the candidate total, a bound on it,
    // until the caller reads the count back.
    DRel finalize_async(Bags &bags, const DRel &against, Buf<uint64_t> &cnt) {
        const uint64_t total = bags.rows();
        DRel d;
        if (total == 0) {
            bags.clear();
            return d;
        }
        Owned cat(ctx);
        const bool grouped = bags.v.size() == 1 && bags.grouped[0] && total < (1ull << 30) && digits &&
                             total / bags.grouped[0] <= SHORT_GROUP_ROWS;
        if (bags.v.size() == 1) {
            cat.reset(bags.v[0].first);
            bags.v.clear();
            bags.grouped.clear();
        } else {
            cat.reset(alloc_keys(ctx, total));
            uint64_t off = 0;
            for (auto &b : bags.v) {
                copy_d2d(ctx, cat.p + off, b.first, b.second);
                off += b.second;
            }
            bags.clear();
        }
        Owned srt(ctx);
        if (grouped) {
            // one bag grouped by its high word: one short-run pass (the digit passes only if a run is long)
            Owned alt(ctx, alloc_keys(ctx, total));
            Buf<uint64_t> sc(ctx, 3);
            fill_u64(ctx, sc.p + 2, total, 1);
            sort_grouped_dev(ctx, cat.p, alt.p, total, sc.p + 2, digits, nullptr, sc.p);
            srt.reset(alt.release());
        } else {
            srt.reset(sort_keys(ctx, cat.release(), total, true, 0, 8, digits));  // consumes cat
        }
        Owned o(ctx, alloc_keys(ctx, total));
        cnt = Buf<uint64_t>(ctx, 1);
        select_unique_diff(ctx, srt.p, total, against.k, against.n, o.p, cnt.p);
        d.n = total;
        d.k = o.release();
        d.owned = true;
        d.version = version_counter++;
        return d;
    }
    DRel finalize(Bags &bags, const DRel &against) {
        Buf<uint64_t> cnt;
        DRel d = finalize_async(bags, against, cnt);
        if (d.k) d.n = read_count(ctx, cnt.p);
        return d;
    }

    DRel merge(const DRel &a, const DRel &b) {
        DRel m;
        m.n = a.n + b.n;
        Owned k(ctx, alloc_keys(ctx, m.n));
        merge_sorted(ctx, a.k, a.n, b.k, b.n, k.p);
        m.k = k.release();
        m.owned = true;
        m.version = version_counter++;
        return m;
    }

    void release(DRel &r) {
        drop_index(r);
        if (r.owned) ctx->free(r.k);
        r = DRel();
    }

    // The first join of a variant whose delta atom comes first and whose other
    // atoms are all EDB (their indexes never change): its count pass can run
    // as soon as the delta exists on the device, before its size is known, so
    // the iteration needs one read-back (delta sizes and these totals together).
    bool precountable(const Rule &r, int occ, int *bpos, int *apos) const {
        if (occ != 0 || r.nb < 2 || !idb[r.b[0].pred]) return false;
        for (int j = 1; j < r.nb; ++j)
            if (idb[r.b[j].pred]) return false;
        const Atom &a0 = r.b[0], &a1 = r.b[1];
        if (a0.v[0] == a0.v[1] || a1.v[0] == a1.v[1]) return false;
        if (!needed_later(r, 1, a0.v[0]) || !needed_later(r, 1, a0.v[1])) return false;
        int ns = 0;
        for (int x = 0; x < 2; ++x)
            for (int y = 0; y < 2; ++y)
                if (a0.v[x] == a1.v[y]) { *bpos = x; *apos = y; ++ns; }
        return ns == 1;
    }

    // seed: every rule once against the current store; delta = new \ old,
    // merged into full
    void seed(std::vector<uint64_t> &deltas) {
        obs.assign(rules.size(), {});
        nov.assign(n_preds, 1.0);
        dlast.assign(n_preds, {0, 0});
        std::vector<Bags> derived = bags_per_pred(ctx, n_preds);
        for (const Rule &r : rules) {
            const DRel *rel[MAX_BODY];
            for (int j = 0; j < r.nb; ++j) rel[j] = &full[r.b[j].pred];
            eval_body(r, rel, derived[r.head], nullptr);
        }
        uint64_t total = 0;
        for (uint32_t p = 0; p < n_preds; ++p) {
            if (!idb[p]) continue;
            DRel d = finalize(derived[p], full[p]);  // full_new \ full_old
            delta[p] = d;  // the driver owns it from here
            note_delta(p, d.n);
            if (d.n) {
                DRel m = merge(full[p], d);
                release(full[p]);
                full[p] = m;
            }
            total += d.n;
        }
        deltas.push_back(total);
    }

    // One iteration with its sizes read back (the variants, Δ' = sort+unique(∪
    // variants) \ R, R ∪= Δ'); returns the iteration's Δ total.
    // rs: the rules with the queue's body order (queue_rules), whose join
    // steps' sizes are recorded for the queue's bounds
    uint64_t iterate_host(uint64_t it, std::vector<uint64_t> &deltas, const std::vector<Rule> &rs) {
        cur_iter = it;
        std::vector<Bags> raw = bags_per_pred(ctx, n_preds);
        for (size_t ri = 0; ri < rs.size(); ++ri) {
            const Rule &r = rs[ri];
            for (int occ = 0; occ < r.nb; ++occ) {
                int p = r.b[occ].pred;
                if (!idb[p] || delta[p].n == 0) continue;
                if (r.delta_at >= 0 && occ != r.delta_at) continue;
                const DRel *rel[MAX_BODY];
                for (int j = 0; j < r.nb; ++j) {
                    int q = r.b[j].pred;
                    rel[j] = (j == occ) ? &delta[q] : &full[q];
                }
                eval_body(r, rel, raw[r.head], nullptr, (int)ri);
            }
        }
        uint64_t total = 0;
        for (uint32_t p = 0; p < n_preds; ++p) {
            if (!idb[p]) continue;
            const uint64_t cand = raw[p].rows();
            DRel d = finalize(raw[p], full[p]);
            release(delta[p]);
            delta[p] = d;
            total += d.n;
            if (cand) nov[p] = (double)d.n / (double)cand;
            note_delta(p, d.n);
        }
        deltas.push_back(total);
        if (trace_on()) fprintf(stderr, "[xlog_hip] iteration %llu: delta %llu\n", (unsigned long long)it,
                                (unsigned long long)total);
        if (total == 0) return 0;
        for (uint32_t p = 0; p < n_preds; ++p) {
            if (!idb[p] || delta[p].n == 0) continue;
            DRel m = merge(full[p], delta[p]);
            release(full[p]);
            full[p] = m;
        }
        return total;
    }

    // ---- queued iterations --------------------------------------------------
    // A plan whose every recursive rule reads one IDB atom, first, and EDB
    // atoms after it (transitive closure and other linear programs): each
    // iteration's variants start from a delta and probe indexes that never
    // change, so whole iterations can be queued with every row count left on
    // the device and one read-back per queue.  Each launch of a queued
    // iteration is sized for a bound the host estimates from the sizes seen so
    // far (every join step's rows out per row in, and the share of each
    // head's candidates that were new); a
    // small check kernel compares each device count with its bound before the
    // launches that rely on it and, when it is exceeded (or a join passes the
    // join-row limit or the single-sort size), raises the queue's stop flag
    // with the iteration's number: every later launch of the queue then
    // returns at once.  The host takes the iterations before it as they are
    // and runs that iteration with its sizes read back (iterate_host: the same
    // operators, which also raise the limit's error), then queues again.
    // Relations and deltas alternate between two buffers per predicate, so a
    // stopped iteration never overwrites the state it started from; an
    // iteration that derives nothing rewrites nothing (its merges are
    // skipped), so the queued iterations after the fixpoint change nothing.
    // A rule whose one IDB atom is not first is evaluated from it: the body
    // starts at that atom and takes, each step, the first remaining atom that
    // shares a variable with those already joined (same-generation's
    // sg(X,Y) :- up(X,P), sg(P,Q), down(Q,Y) runs sg, up, down).  The derived
    // set is the same in any order; only the sizes of intermediate bags
    // differ, so with a join-row limit (defined on the bags of the body's own
    // order, relational.rs:4550-4555) only bodies that start with their IDB
    // atom are queued.  qr receives the rules in the order they run.
    bool queue_rules(std::vector<Rule> &qr) const {
        qr.clear();
        bool any = false;
        for (const Rule &orig : rules) {
            std::vector<int> occs;
            for (int j = 0; j < orig.nb; ++j)
                if (idb[orig.b[j].pred]) occs.push_back(j);
            if (occs.empty()) {
                qr.push_back(orig);  // derives only in the seed
                continue;
            }
            if (orig.nb < 2) return false;
            // one variant per IDB atom (it reads the delta, the other IDB atoms R), its body
            // reordered to start there
            for (int at : occs) {
                Rule r = orig;
                if (at != 0) {
                    // a join-row limit must trip where the unqueued loop's body order trips it
                    if (max_join_rows) return false;
                    bool used[MAX_BODY] = {false, false, false, false};
                    std::vector<int> seen{orig.b[at].v[0], orig.b[at].v[1]};
                    r.b[0] = orig.b[at];
                    used[at] = true;
                    for (int pos = 1; pos < orig.nb; ++pos) {
                        int pick = -1;
                        for (int j = 0; j < orig.nb && pick < 0; ++j) {
                            if (used[j]) continue;
                            for (int v : seen)
                                if (orig.b[j].v[0] == v || orig.b[j].v[1] == v) pick = j;
                        }
                        if (pick < 0) return false;
                        used[pick] = true;
                        r.b[pos] = orig.b[pick];
                        seen.push_back(orig.b[pick].v[0]);
                        seen.push_back(orig.b[pick].v[1]);
                    }
                }
                r.delta_at = 0;
                try {
                    const BodyPlan bp = plan_body(r);
                    for (int j = 1; j < r.nb; ++j)
                        if (bp.step[j].filter) return false;  // two-key steps run in the host loop
                } catch (const Error &) {
                    return false;  // this order has no left-deep plan: the host loop takes the program
                }
                qr.push_back(r);
                any = true;
            }
        }
        return any;
    }

    struct QVariant {
        int ri = 0, head = 0, dpred = 0;  // rule, head predicate, delta predicate (atom 0)
        BodyPlan bp;
        const JoinIndex *J[MAX_BODY] = {};
        int dyn[MAX_BODY] = {-1, -1, -1, -1};  // an IDB atom read in full: its index, rebuilt every iteration
        ProbeJob job[MAX_BODY];
        Owned tmp[MAX_BODY] = {Owned(nullptr), Owned(nullptr), Owned(nullptr), Owned(nullptr)};
        uint32_t tot_slot = 0;  // first of its (nb - 1) join-total slots in an iteration's block
    };

    uint64_t run_queued(uint64_t max_iter, std::vector<uint64_t> &deltas, const std::vector<Rule> &qr) {
        const uint64_t qmax = std::min<uint64_t>(env_u64("XLOG_HIP_JOIN_QUEUE", 8), 64);
        std::vector<int> heads, hidx(n_preds, -1);
        for (uint32_t p = 0; p < n_preds; ++p)
            if (idb[p]) {
                hidx[p] = (int)heads.size();
                heads.push_back((int)p);
            }
        small.assign(n_preds, DRel());
        bitr.clear();
        bitr.resize(n_preds);
        if (obs.size() < qr.size()) obs.resize(qr.size());
        uint64_t it = 0;
        bool retried = false;
        while (it < max_iter) {
            const uint64_t done = run_queue(std::min<uint64_t>(qmax, max_iter - it), it, heads, hidx, deltas, qr);
            if (done == ~0ull) {  // converged inside the queue (it counts the empty iteration)
                bitr_settle_all();
                compact_all();
                return it;
            }
            if (done > 0) {
                retried = false;
                continue;
            }
            // a queue that stopped in its first iteration is queued once more with the bounds its
            // counts gave, before the host takes that iteration
            if (q_learned && !retried) {
                retried = true;
                continue;
            }
            retried = false;
            // an iteration whose queue stopped at once, or one for which no queue fits (one run of R)
            bitr_settle_all();
            compact_all();
            ++it;
            if (iterate_host(it, deltas, qr) == 0) return it;
        }
        cur_iter = it;
        bitr_settle_all();
        throw Error{XLOG_HIP_ITERATION_LIMIT,
                    "Recursive SCC iteration limit (" + std::to_string(max_iter) + ") exceeded"};
    }

    // Queues up to qn iterations after iteration `it`.  Returns the number of
    // iterations it completed (it is advanced by them, deltas extended),
    // or ~0 when the fixpoint was reached inside the queue.  A stop at queue
    // position f > 0 leaves the state after iteration it + f; the caller then
    // continues (the stopped iteration is queued again or run from the host).
    uint64_t run_queue(uint64_t qn, uint64_t &it, const std::vector<int> &heads, const std::vector<int> &hidx,
                       std::vector<uint64_t> &deltas, const std::vector<Rule> &qr) {
        const uint32_t H = (uint32_t)heads.size();
        // R as two sorted runs: the base run full[p] is read, never written, by a queue; the recent run
        // small[p] takes every delta (merge) and is merged into the base run here once it holds more than a
        // quarter of it, so the merges of a queue rewrite the recent run instead of all of R
        for (int p : heads)
            if (!bitr[p].lags && small[p].n > full[p].n / 4) compact((uint32_t)p);
        // the variants (one per IDB atom of a recursive rule, that atom first), the fixed indexes of
        // their EDB atoms, and an index per IDB relation (and column) that a variant reads in full,
        // rebuilt on the device at the start of every iteration from R's two runs
        struct DynIndex : DevIndex {
            Owned rk;  // R in one run (base + recent)
            explicit DynIndex(Ctx *c) : DevIndex(c), rk(c) {}
        };
        std::vector<std::unique_ptr<DynIndex>> dyns;
        auto dyn_of = [&](int pred, int apos) {
            for (size_t i = 0; i < dyns.size(); ++i)
                if (dyns[i]->pred == pred && dyns[i]->col == apos) return (int)i;
            std::unique_ptr<DynIndex> d(new DynIndex(ctx));
            d->pred = pred;
            d->col = apos;
            dyns.push_back(std::move(d));
            return (int)dyns.size() - 1;
        };
        std::vector<std::unique_ptr<QVariant>> vars;
        uint32_t tot_words = 0;
        for (size_t ri = 0; ri < qr.size(); ++ri) {
            const Rule &r = qr[ri];
            if (!idb[r.b[0].pred]) continue;
            bool empty_edb = false;
            for (int j = 1; j < r.nb; ++j) empty_edb = empty_edb || (!idb[r.b[j].pred] && full[r.b[j].pred].n == 0);
            if (empty_edb) continue;  // derives nothing, ever
            std::unique_ptr<QVariant> v(new QVariant());
            for (auto &o : v->tmp) o.ctx = ctx;
            v->ri = (int)ri;
            v->head = r.head;
            v->dpred = r.b[0].pred;
            v->bp = plan_body(r);
            for (int j = 1; j < r.nb; ++j) {
                const int q = r.b[j].pred;
                if (idb[q]) v->dyn[j] = dyn_of(q, v->bp.step[j].apos);
                else v->J[j] = &index_of(full[q], v->bp.step[j].apos);
            }
            v->tot_slot = tot_words;  // offset by the block's header below
            tot_words += (uint32_t)(r.nb - 1);
            vars.push_back(std::move(v));
        }
        // words of an iteration's block: nD[H], nR[H], per head its emit bases (one per variant of
        // the head, then its candidate total), the delta total, the variants' join-step totals
        std::vector<uint32_t> base_off(H), nvar(H, 0), vbase(vars.size());
        for (size_t vi = 0; vi < vars.size(); ++vi) vbase[vi] = nvar[hidx[vars[vi]->head]]++;
        uint32_t words_b = 2 * H;
        for (uint32_t h = 0; h < H; ++h) {
            base_off[h] = words_b;
            words_b += nvar[h] + 1;
        }
        const uint32_t total_off = words_b;
        for (auto &vp : vars) vp->tot_slot += total_off + 1;
        const uint32_t B = total_off + 1 + tot_words;
        auto blk = [&](int64_t k) { return (uint64_t)1 + (uint64_t)(k + 1) * B; };
        if (H > QMAX_HEADS) return 0;
        // a head whose one variant keeps its delta's first column as the high word gets its candidates
        // grouped by it, in ascending order: one short-run pass sorts them (sort_grouped_dev)
        std::vector<char> grouped(H, 0);
        std::vector<int> gsrc(H, -1);  // the delta predicate of a grouped head's variant
        for (uint32_t h = 0; h < H; ++h) grouped[h] = nvar[h] == 1;
        for (auto &vp : vars) {
            grouped[hidx[vp->head]] &= vp->bp.grouped ? 1 : 0;
            gsrc[hidx[vp->head]] = hidx[vp->dpred];
        }
        // A grouped head over a domain of at most 2^17 values takes the group bitmaps instead of the sort
        // and the set difference, reading R's rows from R as a bit matrix (domain^2 / 8 bytes, two copies,
        // when that is at most an eighth of the room left) that each iteration brings up to date.  Such a
        // head that no index of the queue reads in full keeps R only in the matrix (no merges), from queue
        // to queue, until a host iteration or the end of the fixpoint needs R's runs (bitr_settle).
        // XLOG_HIP_GROUP_BITMAP: 0 never; 1 group bitmaps over R's runs (no matrix); 2 the matrix with R's
        // runs merged every iteration; unset or 3 all of it.
        const uint64_t gb_mode = env_u64("XLOG_HIP_GROUP_BITMAP", 3);
        const bool gb_on = gb_mode != 0 && domain && domain <= (1ull << 17);
        const uint32_t bw = (uint32_t)((domain + 63) / 64);
        const uint64_t cells = domain * bw;
        // A head whose candidates are not grouped, over a domain whose bit matrix takes at most 128 MiB,
        // filters its join outputs as they are emitted (XLOG_HIP_JOIN_FILTER=0: never): an output already in
        // R (R's bit matrix, kept like the group bitmaps') or already emitted in the iteration (a bit matrix
        // of the outputs taken, claimed by atomic OR) is dropped, so the candidates are the new rows, each
        // once, and sorted they are the delta.  Every join step before a last one drops its repeated
        // outputs the same way.  (The bags are still counted for the join-row limit.)
        bool filt_on = env_u64("XLOG_HIP_JOIN_FILTER", 1) != 0 && domain && cells * 8 <= (128ull << 20);
        if (filt_on) {  // (R's two copies and the outputs taken per filtered head, one per step before a last)
            uint64_t nm = 0;
            for (uint32_t h = 0; h < H; ++h) nm += grouped[h] ? 0 : 3;
            for (auto &vp : vars) nm += (uint64_t)(qr[vp->ri].nb - 2);
            filt_on = nm * cells * 8 <= device_room(ctx) / 8;
        }
        std::vector<char> mh(H, 0), bm(H, 0), fh(H, 0);  // R as a bit matrix; R only as the matrix; filtered
        for (uint32_t h = 0; h < H; ++h) {
            const bool g = grouped[h] && gb_on && gb_mode >= 2, f = !grouped[h] && filt_on;
            if (!g && !f) continue;
            const int p = heads[h];
            BitR &b = bitr[p];
            if (b.domain != domain) b = BitR();
            if (!b.m[0].p) {
                if (16 * cells > device_room(ctx) / 8) continue;
                b.m[0] = Buf<uint64_t>(ctx, cells);
                b.m[1] = Buf<uint64_t>(ctx, cells);
                b.domain = domain;
            }
            if (!bitr_current((uint32_t)p)) {
                b.cur = 0;
                rows_to_bits(ctx, full[p].k ? full[p].k : b.m[1].p, full[p].n, small[p].k ? small[p].k : b.m[1].p,
                             small[p].n, (uint32_t)domain, b.m[0].p);
                bitr_stamp((uint32_t)p);
            }
            // the other copy starts equal (each iteration writes it from the current one)
            XH_CHECK_HIP(hipMemcpyAsync(b.m[b.cur ^ 1].p, b.m[b.cur].p, cells * sizeof(uint64_t),
                                        hipMemcpyDeviceToDevice, ctx->stream));
            mh[h] = 1;
            fh[h] = f;
            bm[h] = f || gb_mode >= 3;
            for (auto &dp : dyns) bm[h] &= dp->pred != p;
        }
        for (uint32_t h = 0; h < H; ++h)
            if (!bm[h]) bitr_settle((uint32_t)heads[h]);  // this queue reads or merges R's runs
        // every block comes back in one read of the pinned staging
        const uint64_t fit = (Ctx::HOST_STAGE_U64 - 1) / B;  // blocks that fit, the starting one included
        if (fit < 3) return 0;
        qn = std::min<uint64_t>(qn, fit - 1);
        // When every head's delta is shrinking, queue only the iterations the decay predicts until the
        // deltas run out (the last two sizes' ratio per iteration), and one more that derives nothing:
        // launches queued past the fixpoint do no work but still cost their dispatch.
        {
            bool decaying = true;
            double left = 0.0, r = 0.0;
            for (uint32_t h = 0; h < H && decaying; ++h) {
                const auto &d2 = dlast[heads[h]];
                if (d2[1] == 0) continue;
                decaying = d2[0] > 0 && d2[1] < d2[0];
                if (decaying) {
                    left += (double)d2[1];
                    r = std::max(r, (double)d2[1] / (double)d2[0]);
                }
            }
            if (decaying && left > 0.0) {
                uint64_t k = 1;
                for (double e = left * r; e >= 0.5 && k < qn; e *= r) ++k;
                qn = std::min<uint64_t>(qn, k + 1);
            }
        }

        // ---- bounds ------------------------------------------------------------
        // rows out per row in of every join step from its last evaluation (4
        // when never seen); a head's next delta is its candidates times the
        // share of them that was new in its last iteration with candidates
        // (before a step has run: the average run length of the index it probes)
        auto fan = [&](const QVariant &v, int j) {
            const auto &o = obs[v.ri][j];
            if (o.first) return std::max(1.0 / 64.0, (double)o.second / (double)o.first);
            if (v.J[j]) {
                const JoinIndex &J = *v.J[j];
                return J.ix.nruns ? std::max(1.0, (double)J.n / (double)J.ix.nruns) : 1.0;
            }
            // an IDB relation read in full: its rows per distinct value (at most the domain's)
            const int q = qr[v.ri].b[j].pred;
            const double rows = (double)r_rows(q);
            const double keys = std::max(1.0, std::min(rows, domain ? (double)domain : rows));
            return std::max(1.0, rows / keys);
        };
        // per-step margin over the estimates and a floor on every bound; tests shrink both
        // (XLOG_HIP_JOIN_QUEUE_MARGIN_PCT, XLOG_HIP_JOIN_QUEUE_SLACK) to make queues stop
        const double M = (double)env_u64("XLOG_HIP_JOIN_QUEUE_MARGIN_PCT", 125) / 100.0;
        const uint64_t SLACK = env_u64("XLOG_HIP_JOIN_QUEUE_SLACK", 4096), SORT_MAX = (1ull << 30) - 1;
        // Lb[k][h]: bound on the delta iteration k reads; T[k][v][j]: join outputs; Cb[k][h]: candidates;
        // Rb[k][h]: R after iteration k (Rb[-1] exact: stored at index 0, iteration k at k + 1)
        std::vector<std::vector<uint64_t>> Lb, Cb, Rb;
        std::vector<std::vector<std::array<uint64_t, MAX_BODY>>> T;
        Rb.push_back({});  // (bounds of the recent run)
        for (int p : heads) Rb[0].push_back(recent_rows(p));
        std::vector<uint64_t> cur(H);
        for (uint32_t h = 0; h < H; ++h) cur[h] = delta[heads[h]].n;  // exact for the first
        const uint64_t room = device_room(ctx) / 2;
        // every derived value is an input value: a head holds at most domain^2 tuples, so its delta is at
        // most what R leaves of that (the bound of small domains)
        std::vector<uint64_t> dmax(H, ~0ull);
        if (domain && domain <= (1ull << 31))
            for (uint32_t h = 0; h < H; ++h)
                dmax[h] = domain * domain - std::min(domain * domain, r_rows(heads[h]));
        uint64_t q = 0;
        for (; q < qn; ++q) {
            std::vector<uint64_t> lb = cur, cb(H, 0), rb(H, 0);
            std::vector<std::array<uint64_t, MAX_BODY>> tv(vars.size());
            // bounds past one sort's size are clamped to it: a larger count stops the queue there and
            // the host loop (which sorts in pieces) takes that iteration
            for (size_t vi = 0; vi < vars.size(); ++vi) {
                const QVariant &v = *vars[vi];
                const Rule &r = qr[v.ri];
                double t = (double)lb[hidx[v.dpred]];
                for (int j = 1; j < r.nb; ++j) {
                    // a step into an IDB relation read in full yields more rows per row as that
                    // relation grows: its fan scales with R's bound over R at the queue's start
                    double g = 1.0;
                    if (v.dyn[j] >= 0) {
                        const int pq = r.b[j].pred;
                        const double r0 = (double)std::max<uint64_t>(r_rows(pq), 1);
                        g = std::max(1.0, (double)(full[pq].n + Rb.back()[hidx[pq]]) / r0);
                    }
                    t = std::min(t * fan(v, j) * g * M + (double)SLACK, (double)SORT_MAX);
                    // filtered outputs are distinct pairs of the domain (and a last step's not in R); a
                    // filtered step not yet seen takes that bound when its buffer is small beside the room
                    if (filt_on && (j < r.nb - 1 || fh[hidx[v.head]])) {
                        const double cap = (double)(j < r.nb - 1 ? domain * domain
                                                                 : std::max<uint64_t>(dmax[hidx[v.head]], 1));
                        t = obs[v.ri][j].first == 0 && 8.0 * cap * (double)MAX_BODY <= (double)room / 16.0
                                ? cap : std::min(t, cap);
                    }
                    tv[vi][j] = (uint64_t)t;
                }
                cb[hidx[v.head]] += tv[vi][r.nb - 1];
            }
            for (uint32_t h = 0; h < H; ++h) cb[h] = std::min(cb[h], SORT_MAX);
            // next deltas, and R after this iteration
            std::vector<uint64_t> nxt(H);
            for (uint32_t h = 0; h < H; ++h) {
                // (a delta never exceeds its head's candidates)
                const double e = (double)cb[h] * (fh[h] ? 1.0 : nov[heads[h]]);  // (filtered: all new)
                nxt[h] = std::min<uint64_t>(std::max<uint64_t>(e > 1e18 ? (uint64_t)1e18 : (uint64_t)e, SLACK), cb[h]);
                nxt[h] = std::min(nxt[h], dmax[h]);
                rb[h] = Rb.back()[h] + nxt[h];
                if (dmax[h] != ~0ull) rb[h] = std::min(rb[h], Rb[0][h] + dmax[h]);
            }
            // device bytes of the queue's buffers with this iteration in it
            uint64_t bytes = 0;
            for (uint32_t h = 0; h < H; ++h) {
                uint64_t mc = cb[h], mr = bm[h] ? 0 : rb[h];
                for (auto &c : Cb) mc = std::max(mc, c[h]);
                bytes += 8 * (4 * mc + 2 * mr);
            }
            // the per-iteration indexes: R in one run (and sorted by its second column), runs, payloads, table
            for (auto &dp : dyns) {
                const uint64_t nr = full[dp->pred].n + Rb.back()[hidx[dp->pred]];
                const uint64_t keys = std::min(nr, domain ? domain : nr);
                bytes += nr * (24 + (dp->col ? 16 : 0)) + 64 * keys;
            }
            for (size_t vi = 0; vi < vars.size(); ++vi) {
                const Rule &r = qr[vars[vi]->ri];
                for (int j = 1; j < r.nb; ++j) {
                    uint64_t mt = tv[vi][j], ml = j == 1 ? lb[hidx[vars[vi]->dpred]] : tv[vi][j - 1];
                    for (size_t k = 0; k < T.size(); ++k) {
                        mt = std::max(mt, T[k][vi][j]);
                        ml = std::max(ml, j == 1 ? Lb[k][hidx[vars[vi]->dpred]] : T[k][vi][j - 1]);
                    }
                    bytes += 12 * ml + (j < r.nb - 1 ? 8 * mt : 0);
                }
            }
            if (bytes > room) break;
            Lb.push_back(lb);
            T.push_back(tv);
            Cb.push_back(cb);
            Rb.push_back(rb);
            cur = nxt;
        }
        if (q < 1) return 0;
        const uint64_t Q = q;

        // ---- buffers -------------------------------------------------------------
        struct QHead {
            Owned C, Calt, D[2], R[2];  // R: the recent run, alternating
            explicit QHead(Ctx *c) : C(c), Calt(c), D{Owned(c), Owned(c)}, R{Owned(c), Owned(c)} {}
        };
        std::vector<std::unique_ptr<QHead>> qh;
        for (uint32_t h = 0; h < H; ++h) {
            uint64_t mc = 0;
            for (uint64_t k = 0; k < Q; ++k) mc = std::max(mc, Cb[k][h]);
            std::unique_ptr<QHead> x(new QHead(ctx));
            x->C.reset(alloc_keys(ctx, mc));
            x->Calt.reset(alloc_keys(ctx, mc));
            x->D[0].reset(alloc_keys(ctx, mc));
            x->D[1].reset(alloc_keys(ctx, mc));
            x->R[0].reset(alloc_keys(ctx, bm[h] ? 1 : Rb[Q][h]));  // (R only as the matrix: not written)
            x->R[1].reset(alloc_keys(ctx, bm[h] ? 1 : Rb[Q][h]));
            qh.push_back(std::move(x));
        }
        for (size_t vi = 0; vi < vars.size(); ++vi) {
            QVariant &v = *vars[vi];
            const Rule &r = qr[v.ri];
            for (int j = 1; j + 1 < r.nb; ++j) {
                uint64_t mt = 0;
                for (uint64_t k = 0; k < Q; ++k) mt = std::max(mt, T[k][vi][j]);
                v.tmp[j].reset(alloc_keys(ctx, mt));
            }
        }
        for (auto &dp : dyns) {
            DynIndex &d = *dp;
            const uint64_t nr = std::max<uint64_t>(full[d.pred].n + Rb[Q - 1][hidx[d.pred]], 1);
            d.rk.reset(alloc_keys(ctx, nr));
            dev_index_alloc(d, nr);
        }
        const uint64_t words = blk((int64_t)Q);  // word 0 (stop) + Q + 1 blocks
        Buf<uint64_t> qs(ctx, words);
        fill_u64(ctx, qs.p, 0ull, words);
        uint32_t *stop = reinterpret_cast<uint32_t *>(qs.p);
        // block -1: the sizes the queue starts from
        for (uint32_t h = 0; h < H; ++h) {
            fill_u64(ctx, qs.p + blk(-1) + h, delta[heads[h]].n, 1);
            fill_u64(ctx, qs.p + blk(-1) + H + h, recent_rows(heads[h]), 1);
        }
        Buf<uint64_t> gscratch(ctx, 2 * (uint64_t)H);
        Buf<uint64_t> tcount(ctx, 1);  // the size of an empty base run
        fill_u64(ctx, tcount.p, 0ull, 1);
        // the group bitmaps' groups: keys and starts
        std::vector<Buf<uint32_t>> gkey(H);
        std::vector<Buf<uint64_t>> gstart(H);
        std::vector<uint64_t> gbound(H, 0);
        Buf<uint64_t> gcount(ctx, H);
        fill_u64(ctx, gcount.p, 0ull, H);
        for (uint32_t h = 0; h < H && gb_on; ++h) {
            if (!grouped[h]) continue;
            uint64_t mc = 0;
            for (uint64_t k = 0; k < Q; ++k) mc = std::max(mc, Cb[k][h]);
            gbound[h] = std::max<uint64_t>(std::min<uint64_t>(mc, domain), 1);
            gkey[h] = Buf<uint32_t>(ctx, gbound[h]);
            gstart[h] = Buf<uint64_t>(ctx, gbound[h]);
        }
        // iteration k reads R's matrix M(k) and writes M(k + 1) (the two copies alternate): a stopped
        // iteration leaves M(k), R after the last completed one, as it was
        auto mat = [&](uint32_t h, uint64_t k) { BitR &b = bitr[heads[h]]; return b.m[(b.cur + k) & 1].p; };
        // the filters' bit matrices of the outputs taken (zero here; after every iteration the rows taken
        // clear their words again) and their counters, per iteration, variant and step: [0] the outputs
        // taken by a step before the last, [1] the count before the step
        std::vector<Buf<uint64_t>> seen_h(H);
        std::vector<std::array<Buf<uint64_t>, MAX_BODY>> seen_s(vars.size());
        for (uint32_t h = 0; h < H; ++h)
            if (fh[h]) {
                seen_h[h] = Buf<uint64_t>(ctx, cells);
                fill_u64(ctx, seen_h[h].p, 0ull, cells);
            }
        for (size_t vi = 0; vi < vars.size() && filt_on; ++vi)
            for (int j = 1; j + 1 < qr[vars[vi]->ri].nb; ++j) {
                seen_s[vi][j] = Buf<uint64_t>(ctx, cells);
                fill_u64(ctx, seen_s[vi][j].p, 0ull, cells);
            }
        Buf<uint64_t> fcnt(ctx, Q * vars.size() * MAX_BODY * 2);
        fill_u64(ctx, fcnt.p, 0ull, Q * vars.size() * MAX_BODY * 2);

        // ---- the queue -------------------------------------------------------------
        cur_iter = it + 1;
        for (uint64_t k = 0; k < Q; ++k) {
            uint64_t *bk = qs.p + blk((int64_t)k), *bp = qs.p + blk((int64_t)k - 1);
            uint64_t *nD = bk, *nR = bk + H, *total = bk + total_off;
            const uint64_t *pD = bp, *pR = bp + H;
            const uint32_t code = (uint32_t)(k + 1);
            // the indexes over R as it stands after the previous iteration (base run + recent run)
            for (auto &dp : dyns) {
                DynIndex &d = *dp;
                const int p = d.pred, hq = hidx[p];
                const uint64_t nb_ = Rb[k][hq], nr = full[p].n + nb_;
                const uint64_t *rin = k == 0 ? small[p].k : qh[hq]->R[(k - 1) & 1].p;
                if (!rin) rin = qh[hq]->R[1].p;  // an empty run read through its device count
                hipLaunchKernelGGL(k_q_rows, dim3(1), dim3(1), 0, ctx->stream, d.cnt.p, full[p].n, pR + hq, nb_, stop);
                XH_CHECK_HIP(hipGetLastError());
                merge_sorted_dev(ctx, full[p].k ? full[p].k : rin, full[p].n, nullptr, rin, nb_, pR + hq, d.rk.p,
                                 nullptr, stop);
                dev_index_build(d, d.rk.p, nr, stop);
            }
            for (size_t vi = 0; vi < vars.size(); ++vi) {
                QVariant &v = *vars[vi];
                const Rule &r = qr[v.ri];
                const int dh_ = hidx[v.dpred], hh = hidx[v.head];
                const uint64_t *left = k == 0 ? delta[v.dpred].k : qh[dh_]->D[(k - 1) & 1].p;
                const uint64_t *d_left = pD + dh_;
                uint64_t left_bound = Lb[k][dh_];
                if (k == 0 && !left) left_bound = 0;
                uint64_t *base_in = bk + base_off[hh] + vbase[vi];
                for (int j = 1; j < r.nb; ++j) {
                    const JoinPlanStep &st = v.bp.step[j];
                    ProbeJob &job = v.job[j];
                    job = ProbeJob();
                    job.probe = left;
                    job.pcol = st.bpos;
                    const JoinIndex &J = v.J[j] ? *v.J[j] : dyns[v.dyn[j]]->J;
                    job.ix = &J.ix;
                    job.payload = J.payload.p;
                    // the first step's count raises the stop flag itself when the delta it reads
                    // is past the bound its launches are sized for
                    probe_prepare_deferred(ctx, job, left_bound, d_left, stop, j == 1 ? code : 0u);
                    const uint64_t *d_tot = job.toff.p + job.tiles;
                    const bool last = j == r.nb - 1;
                    const int oc[4] = {st.sel[0], st.sel[1], 0, 0};
                    uint64_t *out = last ? qh[hh]->C.p : v.tmp[j].p;
                    if (filt_on && (!last || fh[hh])) {
                        // the bag within the join-row limit; its outputs filtered and appended (a last step's
                        // to the head's candidates), within their buffer
                        uint64_t *fc = fcnt.p + ((k * vars.size() + vi) * MAX_BODY + (uint64_t)j) * 2;
                        uint64_t *taken = last ? bk + base_off[hh] + nvar[hh] : fc;
                        const uint64_t cap = last ? Cb[k][hh] : T[k][vi][j];
                        QFilt qf{d_tot, taken, fc + 1, bk + v.tot_slot + (j - 1), max_join_rows, cap};
                        hipLaunchKernelGGL(k_q_fstart, dim3(1), dim3(1), 0, ctx->stream, qf, stop, code);
                        XH_CHECK_HIP(hipGetLastError());
                        const EmitFilter ef{last ? mat(hh, k) : nullptr, last ? seen_h[hh].p : seen_s[vi][j].p, taken,
                                            cap, bw};
                        probe_emit_dev(ctx, job, d_left, oc, out, nullptr, stop, &ef);
                        hipLaunchKernelGGL(k_q_fend, dim3(1), dim3(1), 0, ctx->stream, qf, stop, code);
                        XH_CHECK_HIP(hipGetLastError());
                        d_left = taken;
                    } else {
                        // the output must fit its buffer (and the launches after it their bounds), a join the
                        // limit, and the candidates one sort
                        QStep qsd{d_tot, last ? base_in : nullptr, last ? base_in + 1 : nullptr,
                                  bk + v.tot_slot + (j - 1), last ? Cb[k][hh] : T[k][vi][j], max_join_rows};
                        hipLaunchKernelGGL(k_q_step, dim3(1), dim3(1), 0, ctx->stream, qsd, stop, code);
                        XH_CHECK_HIP(hipGetLastError());
                        probe_emit_dev(ctx, job, d_left, oc, out, last ? base_in : nullptr, stop);
                        d_left = d_tot;
                    }
                    left = out;
                    left_bound = T[k][vi][j];
                }
                // the filtered steps' outputs clear the bits they took
                for (int j = 1; j + 1 < r.nb && filt_on; ++j)
                    rows_bits(ctx, v.tmp[j].p, fcnt.p + ((k * vars.size() + vi) * MAX_BODY + (uint64_t)j) * 2,
                              T[k][vi][j], bw, seen_s[vi][j].p, true, stop);
            }
            // per head: sort the candidates, keep the unique ones not in R
            for (uint32_t h = 0; h < H; ++h) {
                const int p = heads[h];
                const uint64_t *d_cand = bk + base_off[h] + nvar[h];
                uint64_t *ka = qh[h]->C.p, *kb = qh[h]->Calt.p;
                const uint64_t *big = full[p].k ? full[p].k : qh[h]->R[1].p;
                const uint64_t *rin = k == 0 ? small[p].k : qh[h]->R[(k - 1) & 1].p;
                if (!rin) rin = qh[h]->R[1].p;  // an empty run read through its device count
                if (fh[h]) {
                    // the candidates are the new rows, each once: sorted, they are the delta.  They clear
                    // the bits they took, and R's matrix for the next iteration, M(k + 1) (R before the
                    // previous iteration), takes the previous delta and this one
                    radix_sort_dev(ctx, &ka, &kb, Cb[k][h], d_cand, digits, stop);
                    select_not_value(ctx, ka, Cb[k][h], ~0ull, qh[h]->D[k & 1].p, nD + h, d_cand, stop);
                    rows_bits(ctx, qh[h]->D[k & 1].p, nD + h, Cb[k][h], bw, seen_h[h].p, true, stop);
                    if (k > 0)
                        rows_bits(ctx, qh[h]->D[(k - 1) & 1].p, pD + h, Cb[k - 1][h], bw, mat(h, k + 1), false, stop);
                    rows_bits(ctx, qh[h]->D[k & 1].p, nD + h, Cb[k][h], bw, mat(h, k + 1), false, stop);
                    continue;
                }
                if (gbound[h]) {
                    // per group (one high word, its runs listed), the new values by two LDS bitmaps, then
                    // the groups compacted in order; more groups than the domain stop the queue.  M(k + 1)
                    // first takes the rows of the previous iteration's groups (it holds R before them), then
                    // the group kernel writes this iteration's groups' rows into it
                    if (mh[h] && k > 0)
                        copy_group_rows(ctx, gkey[h].p, gcount.p + h, gbound[h], (uint32_t)domain, mat(h, k),
                                        mat(h, k + 1), stop);
                    select_runs(ctx, ka, Cb[k][h], gkey[h].p, gstart[h].p, gcount.p + h, d_cand, stop, gbound[h]);
                    hipLaunchKernelGGL(k_q_cap, dim3(1), dim3(1), 0, ctx->stream, gcount.p + h, gbound[h], stop, code);
                    XH_CHECK_HIP(hipGetLastError());
                    group_bitmap_diff_dev(ctx, ka, Cb[k][h], d_cand, gkey[h].p, gstart[h].p, gbound[h], gcount.p + h,
                                          big, full[p].n, rin, Rb[k][h], pR + h, (uint32_t)domain, ~0ull, kb,
                                          mh[h] ? mat(h, k) : nullptr, mh[h] ? mat(h, k + 1) : nullptr, stop);
                    select_not_value(ctx, kb, Cb[k][h], ~0ull, qh[h]->D[k & 1].p, nD + h, d_cand, stop);
                    continue;
                }
                // (groups: at most one per delta row read and per domain value)
                if (grouped[h] && Cb[k][h] / group_bound(std::max<uint64_t>(Lb[k][gsrc[h]], 1)) <= SHORT_GROUP_ROWS)
                    ka = sort_grouped_dev(ctx, ka, kb, Cb[k][h], d_cand, digits, stop, gscratch.p + 2 * h);
                else radix_sort_dev(ctx, &ka, &kb, Cb[k][h], d_cand, digits, stop);
                // unique, not in the base run (its size is known) and not in the recent run
                select_unique_diff2_dev(ctx, ka, Cb[k][h], d_cand, big, std::max<uint64_t>(full[p].n, 1),
                                        full[p].n ? nullptr : tcount.p, rin, std::max<uint64_t>(Rb[k][h], 1), pR + h,
                                        qh[h]->D[k & 1].p, nD + h, stop);
            }
            // the delta total, R's new sizes within their bounds
            QEnd qe{nD, pR, nR, total, H, {}};
            for (uint32_t h = 0; h < H; ++h) qe.rcap[h] = bm[h] ? ~0ull : Rb[k + 1][h];
            hipLaunchKernelGGL(k_q_end, dim3(1), dim3(1), 0, ctx->stream, qe, stop, code);
            XH_CHECK_HIP(hipGetLastError());
            // per head: R ∪= Δ' into the other buffer (nothing when the iteration derived nothing)
            for (uint32_t h = 0; h < H; ++h) {
                if (bm[h]) continue;
                const int p = heads[h];
                const uint64_t *rin = k == 0 ? small[p].k : qh[h]->R[(k - 1) & 1].p;
                if (!rin) rin = qh[h]->R[1].p;
                merge_sorted_dev(ctx, rin, Rb[k][h], pR + h, qh[h]->D[k & 1].p, Cb[k][h], nD + h,
                                 qh[h]->R[k & 1].p, total, stop);
            }
        }
        ctx->read_scalars(qs.p, words);
        const uint64_t *hs = ctx->host_scalars;
        const uint32_t stopped = (uint32_t)hs[0];  // 0, or queue position + 1
        const uint64_t complete = stopped ? (uint64_t)stopped - 1 : Q;
        if (trace_on()) {
            fprintf(stderr, "[xlog_hip] join queue after iteration %llu: %llu queued, %llu complete; delta bounds",
                    (unsigned long long)it, (unsigned long long)Q, (unsigned long long)complete);
            for (uint64_t k = 0; k < Q; ++k) fprintf(stderr, " %llu", (unsigned long long)Lb[k][0]);
            fprintf(stderr, "; deltas");
            for (uint64_t k = 0; k < complete; ++k) fprintf(stderr, " %llu", (unsigned long long)hs[blk((int64_t)k)]);
            fprintf(stderr, "\n");
        }

        // ---- the completed iterations ----------------------------------------------------
        int64_t last = -1;  // the last completed queue position
        bool converged = false;
        for (uint64_t k = 0; k < complete; ++k) {
            const uint64_t *bk = hs + blk((int64_t)k);
            const uint64_t *bp = hs + blk((int64_t)k - 1);
            ++it;
            uint64_t tot = 0;
            for (uint32_t h = 0; h < H; ++h) tot += bk[h];
            deltas.push_back(tot);
            for (uint32_t h = 0; h < H; ++h) {
                if (const uint64_t cand = bk[base_off[h] + nvar[h]]) nov[heads[h]] = (double)bk[h] / (double)cand;
                note_delta(heads[h], bk[h]);
            }
            for (auto &vp : vars) {
                const Rule &r = qr[vp->ri];
                uint64_t in = bp[hidx[vp->dpred]];
                for (int j = 1; j < r.nb; ++j) {
                    const uint64_t o = bk[vp->tot_slot + (j - 1)];
                    if (in) obs[vp->ri][j] = {in, o};
                    in = o;
                }
            }
            if (tot == 0) {
                converged = true;
                break;
            }
            last = (int64_t)k;
        }
        // hand the state after the last completed iteration to the driver
        if (last >= 0) {
            const uint64_t *bk = hs + blk(last);
            for (uint32_t h = 0; h < H; ++h) {
                const int p = heads[h];
                if (bm[h]) {
                    // R stays in the matrix (its runs lag it until bitr_settle)
                    bitr[p].rows = r_rows(p) + (bk[H + h] - recent_rows(p));
                    bitr[p].lags = true;
                } else {
                    release(small[p]);
                    small[p].n = bk[H + h];
                    small[p].k = qh[h]->R[last & 1].release();
                    small[p].owned = true;
                    small[p].version = version_counter++;
                }
                if (mh[h]) {
                    bitr[p].cur = (bitr[p].cur + (int)(last + 1)) & 1;
                    bitr_stamp((uint32_t)p);
                }
            }
        }
        if (converged || last >= 0) {
            // the deltas after the last completed iteration (all empty when converged)
            const int64_t kd = converged ? (int64_t)(complete > 0 ? std::min<uint64_t>(complete - 1, Q - 1) : 0) : last;
            const uint64_t *bk = hs + blk(kd);
            for (uint32_t h = 0; h < H; ++h) {
                const int p = heads[h];
                if (converged) {
                    release(delta[p]);
                    continue;
                }
                release(delta[p]);
                delta[p].n = bk[h];
                delta[p].k = qh[h]->D[kd & 1].release();
                delta[p].owned = true;
                delta[p].version = version_counter++;
            }
        }
        // a stopped iteration's counts up to the stop (join totals, and its deltas when the stop came
        // after them) size the next queue's bounds
        q_learned = false;
        if (stopped && !converged) {
            const uint64_t *bk = hs + blk((int64_t)complete);
            const uint64_t *bp = hs + blk((int64_t)complete - 1);
            for (auto &vp : vars) {
                const Rule &r = qr[vp->ri];
                uint64_t in = bp[hidx[vp->dpred]];
                for (int j = 1; j < r.nb; ++j) {
                    const uint64_t o = bk[vp->tot_slot + (j - 1)];
                    if (!o) break;  // the steps after the stop did not run
                    if (in) {
                        obs[vp->ri][j] = {in, o};
                        q_learned = true;
                    }
                    in = o;
                }
            }
            for (uint32_t h = 0; h < H; ++h) {
                const uint64_t cand = bk[base_off[h] + nvar[h]];
                if (cand && bk[h]) {
                    nov[heads[h]] = (double)bk[h] / (double)cand;
                    q_learned = true;
                }
            }
        }
        if (converged) return ~0ull;
        return (uint64_t)(last + 1);
    }

    uint64_t run(uint64_t max_iter, std::vector<uint64_t> &deltas) {
        seed(deltas);
        std::vector<Rule> qr;
        if (env_u64("XLOG_HIP_JOIN_QUEUE", 8) >= 2 && queue_rules(qr)) return run_queued(max_iter, deltas, qr);
        // count jobs of the next iteration's pre-countable first joins, by (rule, occurrence)
        std::map<std::pair<int, int>, std::unique_ptr<ProbeJob>> pre;
        uint64_t it = 0;
        while (it < max_iter) {
            cur_iter = ++it;
            std::vector<Bags> raw = bags_per_pred(ctx, n_preds);
            for (size_t ri = 0; ri < rules.size(); ++ri) {
                const Rule &r = rules[ri];
                for (int occ = 0; occ < r.nb; ++occ) {
                    int p = r.b[occ].pred;
                    if (!idb[p] || delta[p].n == 0) continue;
                    const DRel *rel[MAX_BODY];
                    for (int j = 0; j < r.nb; ++j) {
                        int q = r.b[j].pred;
                        rel[j] = (j == occ) ? &delta[q] : &full[q];
                    }
                    auto pj = pre.find({(int)ri, occ});
                    eval_body(r, rel, raw[r.head], pj != pre.end() ? pj->second.get() : nullptr);
                }
            }
            pre.clear();
            // the new deltas, their counts on the device
            std::vector<Buf<uint64_t>> cnt(n_preds);
            for (uint32_t p = 0; p < n_preds; ++p) {
                if (!idb[p]) continue;
                DRel d = finalize_async(raw[p], full[p], cnt[p]);
                release(delta[p]);
                delta[p] = d;
            }
            // count passes of the next iteration's pre-countable first joins
            for (size_t ri = 0; ri < rules.size(); ++ri) {
                const Rule &r = rules[ri];
                int bpos = 0, apos = 0;
                if (!precountable(r, 0, &bpos, &apos)) continue;
                const DRel &d = delta[r.b[0].pred];
                if (!d.k || full[r.b[1].pred].n == 0) continue;
                const JoinIndex &J = index_of(full[r.b[1].pred], apos);
                std::unique_ptr<ProbeJob> job(new ProbeJob());
                job->probe = d.k;
                job->pcol = bpos;
                job->ix = &J.ix;
                job->payload = J.payload.p;
                probe_prepare_deferred(ctx, *job, d.n, cnt[r.b[0].pred].p);
                pre[{(int)ri, 0}] = std::move(job);
            }
            // one read-back: every delta size and every pre-counted total
            std::vector<const uint64_t *> src;
            for (uint32_t p = 0; p < n_preds; ++p)
                if (idb[p] && delta[p].k) src.push_back(cnt[p].p);
            for (auto &kv : pre) src.push_back(kv.second->toff.p + kv.second->tiles);
            if (!src.empty()) {
                XH_REQUIRE(src.size() <= Ctx::HOST_STAGE_U64, XLOG_HIP_UNSUPPORTED, "fixpoint: too many predicates");
                Buf<uint64_t> gather(ctx, src.size());
                for (size_t q = 0; q < src.size(); ++q) copy_d2d(ctx, gather.p + q, src[q], 1);
                ctx->read_scalars(gather.p, src.size());
            }
            size_t q = 0;
            uint64_t total = 0;
            for (uint32_t p = 0; p < n_preds; ++p) {
                if (!idb[p] || !delta[p].k) continue;
                delta[p].n = ctx->host_scalars[q++];
                total += delta[p].n;
            }
            for (auto &kv : pre) {
                const int p0 = rules[kv.first.first].b[0].pred;
                probe_finish(*kv.second, delta[p0].n, ctx->host_scalars[q++]);
            }
            deltas.push_back(total);
            if (trace_on()) fprintf(stderr, "[xlog_hip] iteration %llu: delta %llu\n", (unsigned long long)it,
                                    (unsigned long long)total);
            if (total == 0) return it;
            for (uint32_t p = 0; p < n_preds; ++p) {
                if (!idb[p] || delta[p].n == 0) continue;
                DRel m = merge(full[p], delta[p]);
                release(full[p]);
                full[p] = m;
            }
        }
        throw Error{XLOG_HIP_ITERATION_LIMIT,
                    "Recursive SCC iteration limit (" + std::to_string(max_iter) + ") exceeded"};
    }

    // The loop of run() over device hash sets, for path-shaped rules of at
    // most three atoms (chains[ri]: rule ri as a path from its first head
    // variable to its second).  The full relation of every IDB predicate also
    // lives in a hash set; a pass runs one expand-and-insert launch per
    // variant (hs_path_insert: the delta atom's rows through the other atoms'
    // run indexes, at most two hops, no intermediate relation), and the tuples
    // a head's launches insert are its next delta: new against R and unique,
    // with no sort, merge-diff or candidate bag.  Pass 0 is the seed (every
    // rule once, its first path atom reading its whole relation: the tuples it
    // inserts are T(R) minus R, run()'s seed).  Up to XLOG_HIP_HASH_QUEUE (8)
    // iterations are queued per read-back: each launch reads its delta's row
    // count on the device, and a step that overflows makes the later queued
    // steps do nothing and is rerun with the host's sizes.  A predicate that
    // some variant reads in full (an IDB atom besides the delta atom) is kept
    // sorted in its full relation for the indexes: a synchronous pass merges
    // its appends, and before each queued step the appends of the step before
    // are sorted and merged and the indexes rebuilt on the device.  The
    // others are collected from their set at the end.
    uint64_t run_hash(uint64_t max_iter, std::vector<uint64_t> &deltas, const std::vector<ChainRule> &chains) {
        XH_REQUIRE(chains.size() == rules.size(), XLOG_HIP_INVALID_ARG, "hash route: one path per rule");
        std::vector<bool> indexed(n_preds, false);
        bool any_indexed = false;
        for (const ChainRule &c : chains) {
            XH_REQUIRE(c.path.size() >= 1 && c.path.size() <= 3, XLOG_HIP_UNSUPPORTED,
                       "hash route: rule bodies of 1 to 3 atoms");
            for (size_t d = 0; d < c.path.size(); ++d) {
                if (!idb[c.path[d].pred]) continue;
                for (size_t j = 0; j < c.path.size(); ++j)
                    if (j != d && idb[c.path[j].pred]) indexed[c.path[j].pred] = any_indexed = true;
            }
        }
        std::vector<HashSet> H(n_preds);
        std::vector<Buf<uint64_t>> dcur(n_preds);  // the current delta rows (sorted only when indexed)
        std::vector<uint64_t> dn(n_preds, 0);
        for (uint32_t p = 0; p < n_preds; ++p) {
            if (!idb[p]) continue;
            hs_init(ctx, H[p], env_u64("XLOG_HIP_HASH_SLOTS", std::max<uint64_t>(4 * full[p].n, 1ull << 16)));
            if (H[p].cap / 2 < full[p].n) hs_grow(ctx, H[p], 4 * full[p].n);
            if (full[p].n) {
                hs_insert_all(ctx, H[p], full[p].k, full[p].n);
                H[p].size = full[p].n;
            }
        }
        struct Var {
            PathInsertArgs a;
            bool copy = false;  // one-atom body: the delta rows themselves (swapped when `swap`)
            bool swap = false;
            double fanout = 1.0;  // expected head tuples per delta row
            int hp[2] = {-1, -1}, hc[2] = {0, 0};  // per hop: the predicate and key column it reads
        };
        // The launch arguments of the variant with the delta at path position d of rule ri (rows left
        // unset), with its hops at the current full relations; false when a hop has no run at all.  In
        // queued steps (queued) a hop into an indexed predicate is left to the index the queue rebuilds
        // on the device before every step.
        auto make_var = [&](size_t ri, int d, Var &v, bool queued = false) -> bool {
            const std::vector<ChainAtom> &path = chains[ri].path;
            const int m = (int)path.size();
            v = Var();
            v.a.delta_swap = path[d].backward ? 1 : 0;
            // a hop through atom j: from x_{j+1} to x_j (left of the delta atom) or from x_j to
            // x_{j+1} (right of it); the stored tuple is (x_j, x_{j+1}) unless backward
            auto hop = [&](int j, bool left, PathHop &h) {
                const bool key_col1 = left != path[j].backward;
                const int slot = &h == &v.a.h1 ? 0 : 1;
                v.hp[slot] = path[j].pred;
                v.hc[slot] = key_col1 ? 1 : 0;
                if (queued && indexed[path[j].pred]) return true;
                const DRel &rel = full[path[j].pred];
                if (rel.n == 0) return false;
                const JoinIndex &J = index_of(rel, key_col1 ? 1 : 0);
                h.table = J.ix.table.p;
                h.mask = J.ix.table_mask;
                int bits = 0;
                while ((1ull << bits) < J.ix.table_mask + 1) ++bits;
                h.bits = bits;
                h.payload = J.payload.p;
                v.fanout *= J.ix.nruns ? (double)J.n / (double)J.ix.nruns : 0.0;
                return J.ix.nruns != 0;
            };
            if (m == 1) {
                v.copy = true;
                v.swap = path[0].backward;
                return true;
            }
            if (m == 2) {  // d = 0: xb -> x2 (right); d = 1: xa -> x0 (left)
                v.a.key1 = d == 0 ? 1 : 0;
                v.a.out0 = d == 0 ? 0 : 2;
                v.a.out1 = d == 0 ? 2 : 1;
                return hop(d == 0 ? 1 : 0, d == 1, v.a.h1);
            }
            if (d == 0) {  // xb -> x2 -> x3
                v.a.key1 = 1;
                v.a.key2 = 2;
                v.a.out0 = 0;
                v.a.out1 = 3;
                return hop(1, false, v.a.h1) && hop(2, false, v.a.h2);
            }
            if (d == 1) {  // xa -> x0 and xb -> x3
                v.a.key1 = 0;
                v.a.key2 = 1;
                v.a.out0 = 2;
                v.a.out1 = 3;
                return hop(0, true, v.a.h1) && hop(2, false, v.a.h2);
            }
            v.a.key1 = 0;  // xa -> x1 -> x0
            v.a.key2 = 2;
            v.a.out0 = 3;
            v.a.out1 = 1;
            return hop(1, true, v.a.h1) && hop(0, true, v.a.h2);
        };
        auto launch = [&](HashSet &h, const Var &v, uint64_t *out, uint64_t limit, unsigned long long *count,
                          unsigned long long *overflow) {
            if (v.copy)
                hs_insert_novel(ctx, h, v.a.delta, v.a.n, out, limit, v.swap ? 1 : 0, count, overflow, &v.a.q);
            else
                hs_path_insert(ctx, h, v.a, out, limit, count, overflow);
        };
        // appends allowed per attempt: the expected candidate count, a bound on the novel tuples
        // (XLOG_HIP_HASH_APPENDS below 2^20 forces small attempts: tests of the rerun path)
        const uint64_t min_want = env_u64("XLOG_HIP_HASH_APPENDS", 1ull << 20);
        // One synchronous pass: every head's variants until none overflows.  appended / out may hold the
        // appends of a queued step that overflowed (kept: those tuples are in the set already).
        auto sync_pass = [&](std::vector<std::vector<Var>> &vars, std::vector<uint64_t> &appended,
                             std::vector<Buf<uint64_t>> &out) {
            std::vector<uint64_t> want(n_preds, 0);
            std::vector<uint32_t> todo;
            for (uint32_t p = 0; p < n_preds; ++p) {
                if (vars[p].empty()) continue;
                // the candidates expected, but at most 4x the set and the delta rows (duplicate-heavy
                // bodies, like the non-linear closure, expand to far more candidates than novel tuples;
                // the rerun protocol covers an estimate that is too small)
                double est = 0, rows = 0;
                for (const Var &v : vars[p]) {
                    est += (double)v.a.n * v.fanout;
                    rows += (double)v.a.n;
                }
                est = std::min(est * 1.25, 4.0 * ((double)H[p].size + rows));
                want[p] = min_want < (1ull << 20) ? min_want : std::max<uint64_t>(min_want, (uint64_t)est + 1024);
                fill_u64(ctx, H[p].flags.p + 1, 0ull, 1);
                fill_u64(ctx, H[p].flags.p + 2, appended[p], 1);
                todo.push_back(p);
            }
            while (!todo.empty()) {
                for (uint32_t p : todo) {
                    HashSet &h = H[p];
                    uint64_t room = h.cap / 2 > h.size + appended[p] ? h.cap / 2 - h.size - appended[p] : 0;
                    if (room < want[p]) {
                        // 4x what this step needs: R keeps growing, and every rehash re-inserts all of it
                        hs_grow(ctx, h, 4 * (h.size + appended[p] + want[p]));
                        room = h.cap / 2 - h.size - appended[p];
                    }
                    const uint64_t limit = appended[p] + std::min(want[p], room);
                    // every launch appends at most HS_APPEND_SLACK past the limit
                    const uint64_t need = limit + (uint64_t)vars[p].size() * HS_APPEND_SLACK;
                    if (out[p].n < need) {
                        Buf<uint64_t> bigger(ctx, need);
                        if (appended[p]) copy_d2d(ctx, bigger.p, out[p].p, appended[p]);
                        out[p] = std::move(bigger);
                    }
                    for (const Var &v : vars[p]) launch(h, v, out[p].p, limit, nullptr, nullptr);
                }
                // one read-back: every head's overflow flag and appended count
                Buf<uint64_t> g(ctx, 2 * todo.size());
                for (size_t t = 0; t < todo.size(); ++t) copy_d2d(ctx, g.p + 2 * t, H[todo[t]].flags.p + 1, 2);
                ctx->read_scalars(g.p, 2 * todo.size());
                std::vector<uint32_t> again;
                for (size_t t = 0; t < todo.size(); ++t) {
                    const uint32_t p = todo[t];
                    appended[p] = ctx->host_scalars[2 * t + 1];
                    if (ctx->host_scalars[2 * t]) {
                        // the limit or a full table stopped a launch: grow and run the head's variants again;
                        // the tuples they inserted are found present and are not appended twice
                        fill_u64(ctx, H[p].flags.p + 1, 0ull, 1);
                        want[p] *= 4;
                        again.push_back(p);
                    }
                }
                todo.swap(again);
            }
        };
        // a finished pass: the appended tuples become the deltas (sorted into full R where indexed)
        auto finish_pass = [&](std::vector<uint64_t> &appended, std::vector<Buf<uint64_t>> &out) {
            uint64_t total = 0;
            for (uint32_t p = 0; p < n_preds; ++p) {
                if (!idb[p]) continue;
                total += appended[p];
                H[p].size += appended[p];
                dn[p] = appended[p];
                if (!appended[p]) {
                    dcur[p] = Buf<uint64_t>();
                    continue;
                }
                if (indexed[p]) {
                    // sorted: the delta joins R for the next pass's indexes
                    uint64_t *sd = sort_keys(ctx, out[p].p, appended[p], false, 0, 8, digits);
                    dcur[p] = Buf<uint64_t>();
                    dcur[p].ctx = ctx;
                    dcur[p].p = sd;
                    dcur[p].n = appended[p];
                    DRel d;
                    d.k = sd;
                    d.n = appended[p];
                    d.owned = false;
                    DRel m = merge(full[p], d);
                    release(full[p]);
                    full[p] = m;
                } else {
                    dcur[p] = std::move(out[p]);
                }
            }
            return total;
        };
        // the variants of a synchronous pass over the current deltas (pass 0: the seed)
        auto pass_vars = [&](bool seed) {
            std::vector<std::vector<Var>> vars(n_preds);
            for (size_t ri = 0; ri < chains.size(); ++ri) {
                const std::vector<ChainAtom> &path = chains[ri].path;
                for (int d = 0; d < (int)path.size(); ++d) {
                    const int q = path[d].pred;
                    if (seed ? (d != 0 || full[q].n == 0) : (!idb[q] || dn[q] == 0)) continue;
                    Var v;
                    if (!make_var(ri, d, v)) continue;
                    v.a.delta = seed ? full[q].k : dcur[q].p;
                    v.a.n = seed ? full[q].n : dn[q];
                    vars[chains[ri].head].push_back(v);
                }
            }
            return vars;
        };
        {  // pass 0, the seed
            std::vector<std::vector<Var>> vars = pass_vars(true);
            std::vector<uint64_t> appended(n_preds, 0);
            std::vector<Buf<uint64_t>> out(n_preds);
            sync_pass(vars, appended, out);
            deltas.push_back(finish_pass(appended, out));
        }
        const uint64_t queue_max = std::min<uint64_t>(env_u64("XLOG_HIP_HASH_QUEUE", 8), 256);
        uint64_t queue = queue_max;
        std::vector<Buf<uint64_t>> spare(n_preds);  // the second delta buffer of the queued steps
        std::vector<uint64_t> cap(n_preds, 0);
        uint64_t it = 0;
        for (;;) {
            XH_REQUIRE(it < max_iter, XLOG_HIP_ITERATION_LIMIT,
                       "Recursive SCC iteration limit (" + std::to_string(max_iter) + ") exceeded");
            uint64_t total_now = 0;
            for (uint32_t p = 0; p < n_preds; ++p) total_now += idb[p] ? dn[p] : 0;
            const uint64_t K = std::min<uint64_t>(queue, max_iter - it);
            if (K >= 2 && total_now) {
                // ---- K queued steps, one read-back ----
                std::vector<std::vector<std::pair<size_t, int>>> by_head(n_preds);  // (rule, delta position)
                std::vector<std::vector<Var>> tmpl(n_preds);
                for (size_t ri = 0; ri < chains.size(); ++ri)
                    for (int d = 0; d < (int)chains[ri].path.size(); ++d) {
                        if (!idb[chains[ri].path[d].pred]) continue;
                        Var v;
                        if (!make_var(ri, d, v, true)) continue;
                        by_head[chains[ri].head].push_back({ri, d});
                        tmpl[chains[ri].head].push_back(v);
                    }
                // delta buffers: ring[j % 2] holds the delta after step j of the batch (ring[0]: the current one)
                std::vector<Buf<uint64_t>> ring[2];
                std::vector<uint64_t> room(n_preds, 0);
                ring[0].resize(n_preds);
                ring[1].resize(n_preds);
                for (uint32_t p = 0; p < n_preds; ++p) {
                    if (!idb[p]) continue;
                    // each step's appends: 4x the delta, growing with the deltas seen (a step past it overflows
                    // and is rerun; XLOG_HIP_HASH_APPENDS below 2^20 fixes it, for tests of that path)
                    cap[p] = min_want < (1ull << 20) ? min_want : std::max<uint64_t>({cap[p], 4 * dn[p], 1ull << 16});
                    const uint64_t need = std::max(cap[p] + (uint64_t)tmpl[p].size() * HS_APPEND_SLACK, dn[p]);
                    if (dcur[p].n >= need) {
                        ring[0][p] = std::move(dcur[p]);
                    } else {
                        ring[0][p] = Buf<uint64_t>(ctx, need);
                        if (dn[p]) copy_d2d(ctx, ring[0][p].p, dcur[p].p, dn[p]);
                        dcur[p] = Buf<uint64_t>();
                    }
                    ring[1][p] = spare[p].n >= need ? std::move(spare[p]) : Buf<uint64_t>(ctx, need);
                    HashSet &h = H[p];
                    // room for two steps' appends at least; the steps' appends together stop at half load
                    // (QueuedStep::room), and a step cut short by it is one more overflow and a rerun
                    if (!tmpl[p].empty() && h.cap / 2 < h.size + 2 * cap[p]) hs_grow(ctx, h, 4 * (h.size + 2 * cap[p]));
                    room[p] = h.cap / 2 > h.size ? h.cap / 2 - h.size : 0;
                }
                const uint32_t P = n_preds;
                Buf<uint64_t> cnt(ctx, (K + 1) * P), ovf(ctx, K + 1);
                fill_u64(ctx, cnt.p, 0ull, (K + 1) * P);
                fill_u64(ctx, ovf.p, 0ull, K + 1);
                unsigned long long *ucnt = reinterpret_cast<unsigned long long *>(cnt.p);
                unsigned long long *uovf = reinterpret_cast<unsigned long long *>(ovf.p);
                // An indexed predicate's R after step j is R_j = R_{j-1} ∪ (step j's appends): before step
                // j >= 2 the appends of step j-1 are sorted (in their ring buffer: a permutation of the same
                // rows) and merged into the other of two buffers, and the indexes that the variants' hops
                // read are rebuilt from it; after the last step R_K is merged once more.  Every count stays
                // on the device; a step that overflowed stops all of this (k_any_set).
                struct QR {
                    Owned RB[2], srt_alt;
                    Buf<uint64_t> dR;  // [j]: rows of R_j (R_0: full)
                    uint64_t bound = 0;
                    explicit QR(Ctx *c) : RB{Owned(c), Owned(c)}, srt_alt(c) {}
                };
                std::vector<std::unique_ptr<QR>> qrel(n_preds);
                std::vector<std::unique_ptr<DevIndex>> devs;
                Buf<uint32_t> stp(ctx, 1);
                fill_u32(ctx, stp.p, 0u, 1);
                for (uint32_t p = 0; p < n_preds; ++p)
                    for (size_t t = 0; t < tmpl[p].size(); ++t)
                        for (int slot = 0; slot < 2; ++slot) {
                            Var &v = tmpl[p][t];
                            const int q = v.hp[slot];
                            if (q < 0 || !indexed[q]) continue;
                            if (!qrel[q]) {
                                std::unique_ptr<QR> x(new QR(ctx));
                                x->bound = full[q].n + K * cap[q];
                                x->RB[0].reset(alloc_keys(ctx, x->bound));
                                x->RB[1].reset(alloc_keys(ctx, x->bound));
                                x->srt_alt.reset(alloc_keys(ctx, cap[q]));
                                x->dR = Buf<uint64_t>(ctx, K + 1);
                                fill_u64(ctx, x->dR.p, full[q].n, 1);
                                qrel[q] = std::move(x);
                            }
                            DevIndex *d = nullptr;
                            for (auto &e : devs)
                                if (e->pred == q && e->col == v.hc[slot]) d = e.get();
                            if (!d) {
                                devs.emplace_back(new DevIndex(ctx));
                                d = devs.back().get();
                                d->pred = q;
                                d->col = v.hc[slot];
                                dev_index_alloc(*d, qrel[q]->bound);
                            }
                            PathHop &h = slot ? v.a.h2 : v.a.h1;
                            h.table = d->J.ix.table.p;
                            h.mask = d->J.ix.table_mask;
                            h.bits = __builtin_ctzll(d->J.ix.table_mask + 1);
                            h.payload = d->J.payload.p;
                        }
                // R_{j-1} and the indexes over it, before step j (j = K + 1: R_K only)
                auto refresh = [&](uint64_t j) {
                    if (j >= 2) {
                        hipLaunchKernelGGL(k_any_set, dim3(1), dim3(1), 0, ctx->stream, uovf + 1, (uint32_t)(j - 1),
                                           stp.p);
                        XH_CHECK_HIP(hipGetLastError());
                    }
                    for (uint32_t q = 0; q < n_preds; ++q) {
                        if (!qrel[q]) continue;
                        QR &x = *qrel[q];
                        const uint64_t *r = full[q].k;  // R_{j-1}
                        uint64_t rn = full[q].n;
                        if (j >= 2) {
                            // the appends of step j - 1, sorted where they lie; merged with R_{j-2}
                            uint64_t *ka = ring[(j - 1) % 2][q].p, *kb = x.srt_alt.p;
                            const uint64_t *dapp = cnt.p + (j - 1) * P + q;
                            radix_sort_dev(ctx, &ka, &kb, cap[q], dapp, digits, stp.p);
                            const uint64_t *prev = j == 2 ? full[q].k : x.RB[(j - 2) % 2].p;
                            const uint64_t prev_n = full[q].n + (j - 2) * cap[q];
                            uint64_t *dst = x.RB[(j - 1) % 2].p;
                            merge_sorted_dev(ctx, prev ? prev : ka, prev_n, j == 2 ? nullptr : x.dR.p + (j - 2), ka,
                                             cap[q], dapp, dst, nullptr, stp.p);
                            hipLaunchKernelGGL(k_add_rows, dim3(1), dim3(1), 0, ctx->stream, x.dR.p + (j - 1),
                                               x.dR.p + (j - 2), dapp, cap[q], stp.p);
                            XH_CHECK_HIP(hipGetLastError());
                            r = dst;
                            rn = prev_n + cap[q];
                        }
                        if (j > K) continue;
                        for (auto &e : devs) {
                            if (e->pred != (int)q) continue;
                            copy_d2d(ctx, e->cnt.p, x.dR.p + (j - 1), 1);
                            dev_index_build(*e, r, rn, stp.p);
                        }
                    }
                };
                for (uint64_t j = 1; j <= K; ++j) {
                    refresh(j);
                    for (uint32_t p = 0; p < n_preds; ++p) {
                        for (size_t t = 0; t < tmpl[p].size(); ++t) {
                            Var v = tmpl[p][t];
                            const int q = chains[by_head[p][t].first].path[by_head[p][t].second].pred;
                            if (j == 1 && dn[q] == 0) continue;
                            v.a.delta = ring[(j - 1) % 2][q].p;
                            v.a.n = j == 1 ? dn[q] : cap[q];
                            v.a.q.d_n = j == 1 ? nullptr : cnt.p + (j - 1) * P + q;
                            v.a.q.stop = uovf + 1;
                            v.a.q.prior = ucnt + P + p;
                            v.a.q.nprior = (int)(j - 1);
                            v.a.q.stride = (int)P;
                            v.a.q.room = room[p];
                            launch(H[p], v, ring[j % 2][p].p, cap[p], ucnt + j * P + p, uovf + j);
                        }
                    }
                }
                refresh(K + 1);
                Buf<uint64_t> g(ctx, K * P + K);
                copy_d2d(ctx, g.p, cnt.p + P, K * P);
                copy_d2d(ctx, g.p + K * P, ovf.p + 1, K);
                ctx->read_scalars(g.p, K * P + K);
                std::vector<uint64_t> hc(ctx->host_scalars, ctx->host_scalars + K * P + K);
                uint64_t j0 = 0;  // the first step that overflowed (0: none)
                bool done = false;
                uint64_t j = 1;
                for (; j <= K; ++j) {
                    if (hc[K * P + j - 1]) {
                        j0 = j;
                        break;
                    }
                    uint64_t total = 0;
                    for (uint32_t p = 0; p < n_preds; ++p)
                        if (idb[p]) {
                            total += hc[(j - 1) * P + p];
                            H[p].size += hc[(j - 1) * P + p];
                            if (min_want >= (1ull << 20)) cap[p] = std::max(cap[p], 2 * hc[(j - 1) * P + p]);
                        }
                    ++it;
                    deltas.push_back(total);
                    if (total == 0) {
                        done = true;
                        break;
                    }
                }
                // the delta of the last complete step becomes the current one
                const uint64_t last = j0 ? j0 - 1 : K;
                if (trace_on())
                    fprintf(stderr, "[xlog_hip] hash queue of %llu steps: %llu complete%s%s\n", (unsigned long long)K,
                            (unsigned long long)(j0 ? j0 - 1 : (done ? j : K)), j0 ? ", one overflowed" : "",
                            done ? ", converged" : "");
                // an indexed predicate's R after that step (R_0: full as it was); at convergence R_K, which
                // the steps after the empty one left unchanged
                for (uint32_t q = 0; q < n_preds; ++q) {
                    if (!qrel[q] || last == 0) continue;
                    uint64_t rn = full[q].n;
                    for (uint64_t t = 1; t <= last; ++t) rn += hc[(t - 1) * P + q];
                    DRel m;
                    m.n = rn;
                    m.k = qrel[q]->RB[last % 2].release();
                    m.owned = true;
                    m.version = version_counter++;
                    release(full[q]);
                    full[q] = m;
                }
                if (done) break;
                for (uint32_t p = 0; p < n_preds; ++p) {
                    if (!idb[p]) continue;
                    if (last) dn[p] = hc[(last - 1) * P + p];
                    dcur[p] = std::move(ring[last % 2][p]);
                    spare[p] = std::move(ring[(last + 1) % 2][p]);
                }
                if (!j0) {
                    queue = std::min<uint64_t>(queue_max, queue * 2);
                    continue;
                }
                // step j0 overflowed: rerun it with the host's sizes, keeping what it appended (in spare)
                XH_REQUIRE(it < max_iter, XLOG_HIP_ITERATION_LIMIT,
                           "Recursive SCC iteration limit (" + std::to_string(max_iter) + ") exceeded");
                cur_iter = ++it;
                std::vector<std::vector<Var>> vars = pass_vars(false);
                std::vector<uint64_t> appended(n_preds, 0);
                std::vector<Buf<uint64_t>> out(n_preds);
                for (uint32_t p = 0; p < n_preds; ++p) {
                    if (!idb[p]) continue;
                    appended[p] = hc[(j0 - 1) * P + p];
                    out[p] = std::move(spare[p]);
                }
                sync_pass(vars, appended, out);
                for (uint32_t p = 0; p < n_preds; ++p)
                    if (idb[p] && min_want >= (1ull << 20)) cap[p] = std::max(cap[p], 2 * appended[p]);
                const uint64_t total = finish_pass(appended, out);
                deltas.push_back(total);
                queue = std::max<uint64_t>(2, j0);
                if (total == 0) break;
                continue;
            }
            // ---- one synchronous iteration ----
            cur_iter = ++it;
            std::vector<std::vector<Var>> vars = pass_vars(false);
            std::vector<uint64_t> appended(n_preds, 0);
            std::vector<Buf<uint64_t>> out(n_preds);
            sync_pass(vars, appended, out);
            const uint64_t total = finish_pass(appended, out);
            deltas.push_back(total);
            if (total == 0) break;
        }
        // predicates not kept sorted: their sets, sorted once
        for (uint32_t p = 0; p < n_preds; ++p) {
            if (!idb[p] || indexed[p]) continue;
            DRel f;
            f.n = H[p].size;
            if (f.n) {
                uint64_t *all = static_cast<uint64_t *>(ctx->alloc(f.n * sizeof(uint64_t)));
                uint64_t got = 0;
                try {
                    got = hs_collect(ctx, H[p], all);
                    XH_REQUIRE(got == f.n, XLOG_HIP_DEVICE_ERROR,
                               "hash set holds " + std::to_string(got) + " tuples, expected " + std::to_string(f.n));
                } catch (...) {
                    ctx->free(all);
                    throw;
                }
                H[p] = HashSet();
                f.k = sort_keys(ctx, all, got, true, 0, 8, digits);  // consumes all
                f.owned = true;
            }
            f.version = version_counter++;
            release(full[p]);
            full[p] = f;
        }
        return it;
    }
};

// TC plan shape: head(A,B) :- E(A,B).  head(A,C) :- head(A,B), E(B,C).
bool tc_shape(const std::vector<Rule> &rules, int *edge_pred, int *head_pred) {
    if (rules.size() != 2) return false;
    const Rule *base = nullptr, *rec = nullptr;
    for (const Rule &r : rules) (r.nb == 1 ? base : rec) = &r;
    if (!base || !rec || rec->nb != 2 || base->head != rec->head) return false;
    int E = base->b[0].pred, H = base->head;
    if (E == H) return false;
    if (!(base->hv[0] == base->b[0].v[0] && base->hv[1] == base->b[0].v[1] && base->hv[0] != base->hv[1])) return false;
    const Atom &x = rec->b[0], &y = rec->b[1];
    if (x.pred != H || y.pred != E) return false;
    int A = x.v[0], B = x.v[1], C = y.v[1];
    if (y.v[0] != B || A == B || B == C || A == C) return false;
    return rec->hv[0] == A && rec->hv[1] == C;
}

// Chain plans: in every rule the body atoms form a simple path from the first
// head variable to the second (each atom read forward or backward), e.g.
// Andersen's  pointsTo(P,O) :- store(V,W), pointsTo(V,P), pointsTo(W,O)  is
// P -pointsTo^T-> V -store-> W -pointsTo-> O.
bool chain_shape(const std::vector<Rule> &rules, std::vector<ChainRule> &out) {
    out.clear();
    for (const Rule &r : rules) {
        if (r.hv[0] == r.hv[1]) return false;
        ChainRule c;
        c.head = r.head;
        bool used[MAX_BODY] = {false, false, false, false};
        int cur = r.hv[0];
        std::vector<int> seen{cur};
        for (int step = 0; step < r.nb; ++step) {
            int pick = -1;
            bool back = false;
            for (int j = 0; j < r.nb; ++j) {
                const Atom &a = r.b[j];
                if (a.v[0] == a.v[1]) return false;
                if (used[j] || (a.v[0] != cur && a.v[1] != cur)) continue;
                if (pick >= 0) return false;  // the path branches
                pick = j;
                back = a.v[1] == cur;
            }
            if (pick < 0) return false;
            used[pick] = true;
            cur = back ? r.b[pick].v[0] : r.b[pick].v[1];
            for (int v : seen)
                if (v == cur) return false;
            seen.push_back(cur);
            c.path.push_back(ChainAtom{r.b[pick].pred, back});
        }
        if (cur != r.hv[1]) return false;
        out.push_back(c);
    }
    return !out.empty();
}

}  // namespace

// a predicate that is the head of some rule
static bool idb_of(const std::vector<Rule> &rules, int pred) {
    for (const Rule &r : rules)
        if (r.head == pred) return true;
    return false;
}

// canonical keys of an input relation for the driver
// Canonical keys of a fixpoint input; for a relation that must be sorted the
// row count stays on the device (*d_count) and d.n is the input's row count,
// a bound, until the caller reads it back.
static DRel canon_drel_async(Ctx *ctx, const xlog_hip_rel *r, uint64_t *d_count, uint32_t known_digits) {
    DRel d;
    if (!r || r->rows == 0) return d;
    XH_REQUIRE(r->arity == 2, XLOG_HIP_TYPE_MISMATCH, "fixpoint: every predicate must have arity 2");
    if (r->flags & REL_CANONICAL) {
        d.k = r->w[0];
        d.n = r->rows;
        d.owned = false;
        return d;
    }
    uint64_t *u;
    sort_unique_keys_async(ctx, r->w[0], r->rows, &u, d_count, known_digits);
    d.n = r->rows;
    d.k = u;
    d.owned = true;
    return d;
}

// Device bytes an operation may still take: the free device memory, within
// the context's budget when one is set.
uint64_t device_room(Ctx *ctx) {
    size_t free_b = 0, total_b = 0;
    XH_CHECK_HIP(hipMemGetInfo(&free_b, &total_b));
    return std::min<uint64_t>((uint64_t)free_b + ctx->pool->bytes_cached(), ctx->pool->headroom());
}

// The dense chain route (chain_fixpoint) when the plan is made of chain rules
// over at most 2^17 ids whose bit matrices fit in half the free device
// memory; false (nothing done) when the join route should run instead, an
// error when the bitmap route was requested and cannot run.  canon: every
// predicate's relation, sorted and unique (read, not consumed); domain: the
// largest id + 1 (0 when every relation is empty).
static bool run_chain_route(Ctx *ctx, const std::vector<Rule> &rules, uint32_t n_preds, const std::vector<DRel> &canon,
                            uint64_t domain, uint64_t route, uint64_t max_iter, xlog_hip_rel **out,
                            uint64_t *iterations, std::vector<uint64_t> &deltas, xlog_hip_fixpoint_stats *stats) {
    std::vector<ChainRule> chains;
    bool chain = route != XLOG_HIP_ROUTE_JOIN && chain_shape(rules, chains);
    XH_REQUIRE(chain || route != XLOG_HIP_ROUTE_BITMAP, XLOG_HIP_UNSUPPORTED,
               "bitmap route needs chain rules (body atoms forming a path between the head variables)");
    if (!chain) return false;
    std::vector<char> idb(n_preds, 0);
    for (const Rule &r : rules) idb[r.head] = 1;
    std::vector<uint64_t *> res;
    auto release = [&]() {
        for (uint64_t *q : res)
            if (q) ctx->free(q);
        res.clear();
    };
    try {
        const bool fits = domain >= 1 && domain <= (1ull << 17) &&
                          chain_fixpoint_bytes(chains, idb, (uint32_t)domain) <= device_room(ctx) / 2;
        XH_REQUIRE(fits || route != XLOG_HIP_ROUTE_BITMAP, XLOG_HIP_UNSUPPORTED,
                   "bitmap route needs 1..2^17 ids and room for the bit matrices");
        if (!fits) return false;
        std::vector<const uint64_t *> keys(n_preds);
        std::vector<uint64_t> rows(n_preds), res_n;
        for (uint32_t p = 0; p < n_preds; ++p) {
            keys[p] = canon[p].k;
            rows[p] = canon[p].n;
        }
        chain_fixpoint(ctx, chains, n_preds, idb, keys, rows, (uint32_t)domain, max_iter, res, res_n, iterations,
                       deltas);
        for (uint32_t p = 0; p < n_preds; ++p) {
            if (!idb[p]) continue;
            out[p] = res_n[p] ? rel_adopt(ctx, 2, res_n[p], res[p], nullptr, REL_CANONICAL) : rel_new(ctx, 2, 0);
            res[p] = nullptr;
            out[p]->flags = REL_CANONICAL;
        }
    } catch (...) {
        release();
        for (uint32_t p = 0; p < n_preds; ++p)
            if (out[p]) {
                rel_free(out[p]);
                out[p] = nullptr;
            }
        if (stats) stats->iterations = deltas.empty() ? 0 : deltas.size() - 1;
        throw;
    }
    release();
    return true;
}

static void run_fixpoint_impl(Ctx *ctx, const int32_t *plan, uint32_t n_preds, const xlog_hip_rel *const *rels,
                              xlog_hip_rel **out, xlog_hip_fixpoint_stats *stats, std::vector<uint64_t> &deltas,
                              uint64_t &reached) {
    XH_REQUIRE(n_preds >= 1 && n_preds <= 256, XLOG_HIP_INVALID_ARG, "n_preds must be 1..256");
    XH_REQUIRE(rels && out, XLOG_HIP_INVALID_ARG, "rels / out is NULL");
    std::vector<Rule> rules = parse_plan(plan, n_preds);
    uint64_t max_iter = (stats && stats->max_iterations) ? stats->max_iterations : 1000000ull;
    uint64_t route = stats ? stats->route : XLOG_HIP_ROUTE_AUTO;
    for (uint32_t p = 0; p < n_preds; ++p) out[p] = nullptr;
    for (uint32_t p = 0; p < n_preds; ++p)
        XH_REQUIRE(!rels[p] || rels[p]->arity == 2, XLOG_HIP_TYPE_MISMATCH, "fixpoint: every predicate must have arity 2");
    XH_CHECK_HIP(hipEventRecord(ctx->ev_a, ctx->stream));
    uint64_t iterations = 0;

    int E = -1, H = -1;
    bool tc = tc_shape(rules, &E, &H);
    if (tc) {
        for (const Rule &r : rules) if (r.nb == 1) { E = r.b[0].pred; H = r.head; }
    }
    bool head_empty = tc && (!rels[H] || rels[H]->rows == 0);
    // path-shaped rules of up to three atoms can also run over hash sets (Driver::run_hash)
    std::vector<ChainRule> paths;
    bool short_paths = chain_shape(rules, paths);
    for (const ChainRule &c : paths) short_paths = short_paths && c.path.size() <= 3;
    XH_REQUIRE(route != XLOG_HIP_ROUTE_HASH || short_paths, XLOG_HIP_UNSUPPORTED,
               "hash route needs rule bodies of 1 to 3 atoms forming a path between the head variables");
    // every relation sorted and unique once, and the largest id (read back first) for every route: the bitmap
    // routes' domain, and the digits the sorts (these and those inside the join and hash routes' loops) vary in
    struct Canon {
        Ctx *ctx;
        std::vector<DRel> d;
        ~Canon() {
            for (DRel &r : d)
                if (r.owned) ctx->free(r.k);
        }
    } canon{ctx, std::vector<DRel>(n_preds)};
    uint64_t nv = 0;  // max id + 1 (up to 2^32; 0 when every relation is empty)
    {
        // Two read-backs: the largest id of the raw inputs (an input's ids are its canonical form's), which
        // gives the digits the sorts can vary in, so that every relation sorts without reading its histograms
        // back; then the canonical row counts, together.
        Buf<uint64_t> sc(ctx, 1 + (uint64_t)n_preds);  // [0]: the largest id (low half), [1 + p]: row counts
        fill_u64(ctx, sc.p, 0ull, 1 + (uint64_t)n_preds);
        uint64_t any = 0;
        for (uint32_t p = 0; p < n_preds; ++p)
            if (rels[p] && rels[p]->rows) {
                any += rels[p]->rows;
                max_u32_of_packed(ctx, rels[p]->w[0], rels[p]->rows, reinterpret_cast<unsigned int *>(sc.p));
            }
        if (any) {
            ctx->read_scalars(sc.p, 1);
            nv = (uint64_t)(uint32_t)ctx->host_scalars[0] + 1;
            // (sorts large enough for the high-word route keep reading their histograms)
            const uint32_t maxid = (uint32_t)(nv - 1);
            const int bits = maxid ? 32 - __builtin_clz(maxid) : 0;
            const uint32_t nd = (uint32_t)(bits + 7) / 8;  // bytes per column
            const uint32_t digits = nd ? (((1u << nd) - 1u) | (((1u << nd) - 1u) << 4)) : 1u;
            for (uint32_t p = 0; p < n_preds; ++p)
                canon.d[p] = canon_drel_async(ctx, rels[p], sc.p + 1 + p,
                                              rels[p] && rels[p]->rows >= (1ull << 22) ? 0u : digits);
            ctx->read_scalars(sc.p + 1, (uint64_t)n_preds);
            for (uint32_t p = 0; p < n_preds; ++p)
                if (canon.d[p].owned) canon.d[p].n = ctx->host_scalars[p];
        }
    }
    bool bitmap = tc && head_empty && route != XLOG_HIP_ROUTE_JOIN && route != XLOG_HIP_ROUTE_HASH &&
                  nv <= (1ull << 17);
    if (bitmap && route == XLOG_HIP_ROUTE_AUTO) {
        // AUTO leaves it when its bit matrices would take more than half the room (a budget, or a busy device)
        std::vector<ChainRule> tcc{ChainRule{H, {ChainAtom{E, false}}}, ChainRule{H, {ChainAtom{E, false}, ChainAtom{H, false}}}};
        std::vector<char> idb1(n_preds, 0);
        idb1[H] = 1;
        bitmap = chain_fixpoint_bytes(tcc, idb1, (uint32_t)std::max<uint64_t>(nv, 1)) <= device_room(ctx) / 2;
    }
    const DRel &edges = tc ? canon.d[E] : canon.d[0];
    if (bitmap) {
        // With the head empty, Δ of iteration k is the set of pairs at shortest distance k + 1 whether the
        // step is Δ ∘ edge (the plan as written) or edge ∘ Δ: a shortest path of length k + 2 splits off its
        // last edge or its first edge, and every other derivation lies in R.  So the left-linear chain
        //   reach(X,Z) :- edge(X,Y), reach(Y,Z)
        // gives the same relation, iteration count and Δ sizes, and its product gathers whole Δ rows
        // (CSR left, bitmap right) instead of expanding adjacency lists id by id.
        uint64_t *res = nullptr, n = 0;
        try {
            if (nv == 0) {  // no edges: the seed and the one empty iteration
                deltas.assign(2, 0);
                iterations = 1;
            } else {
                std::vector<ChainRule> chains{ChainRule{H, {ChainAtom{E, false}}},
                                              ChainRule{H, {ChainAtom{E, false}, ChainAtom{H, false}}}};
                std::vector<char> idb(n_preds, 0);
                idb[H] = 1;
                std::vector<const uint64_t *> keys(n_preds, nullptr);
                std::vector<uint64_t> rows(n_preds, 0), res_n;
                keys[E] = edges.k;
                rows[E] = edges.n;
                std::vector<uint64_t *> r;
                chain_fixpoint(ctx, chains, n_preds, idb, keys, rows, (uint32_t)nv, max_iter, r, res_n, &iterations,
                               deltas);
                res = r[H];
                n = res_n[H];
            }
        } catch (...) {
            if (stats) stats->iterations = deltas.empty() ? 0 : deltas.size() - 1;
            throw;
        }
        out[H] = n ? rel_adopt(ctx, 2, n, res, nullptr, REL_CANONICAL) : rel_new(ctx, 2, 0);
        out[H]->flags = REL_CANONICAL;
        if (stats) stats->route = XLOG_HIP_ROUTE_BITMAP;
    } else if (route != XLOG_HIP_ROUTE_HASH &&
               run_chain_route(ctx, rules, n_preds, canon.d, nv, route, max_iter, out, &iterations, deltas, stats)) {
        if (stats) stats->route = XLOG_HIP_ROUTE_BITMAP;
    } else {
        // Path-shaped plans the bitmap route does not take run over hash sets under AUTO, except (1) when a
        // join-row limit is set (the limit is defined on the join route's bags) and (2) when a three-atom
        // rule reads two or more IDB atoms (Andersen's load and store rules): its two-hop expansions then
        // enumerate every path through the IDB relation's hubs, duplicates included, where the join route
        // deduplicates the first join's pairs (measured at 10,000 variables: 4.5 s against 1.4 s).
        bool hub_paths = false;
        for (const Rule &r : rules) {
            int n_idb = 0;
            for (int j = 0; j < r.nb; ++j) n_idb += idb_of(rules, r.b[j].pred) ? 1 : 0;
            hub_paths = hub_paths || (r.nb == 3 && n_idb >= 2);
        }
        const bool use_hash =
            short_paths && (route == XLOG_HIP_ROUTE_HASH ||
                            (route == XLOG_HIP_ROUTE_AUTO && !(stats && stats->max_join_rows) && !hub_paths));
        Driver drv{ctx, rules, n_preds, std::vector<bool>(n_preds, false), std::vector<DRel>(n_preds),
                   std::vector<DRel>(n_preds)};
        for (const Rule &r : rules) drv.idb[r.head] = true;
        drv.max_join_rows = stats ? stats->max_join_rows : 0;
        for (uint32_t p = 0; p < n_preds; ++p) {
            drv.full[p] = canon.d[p];  // the driver owns them now
            canon.d[p].owned = false;
            drv.full[p].version = drv.version_counter++;
        }
        {
            // Every derived value comes from the inputs, so the largest input id bounds the digits a packed
            // tuple can vary in: sorts inside the loop run those passes without reading histograms back.
            const uint32_t maxid = nv ? (uint32_t)(nv - 1) : 0u;
            const int bits = maxid ? 32 - __builtin_clz(maxid) : 0;
            const uint32_t nd = (uint32_t)(bits + 7) / 8;  // bytes per column
            drv.digits = nd ? (((1u << nd) - 1u) | (((1u << nd) - 1u) << 4)) : 1u;
            drv.domain = nv;
        }
        if (stats) stats->route = use_hash ? XLOG_HIP_ROUTE_HASH : XLOG_HIP_ROUTE_JOIN;  // also on failure
        try {
            iterations = use_hash ? drv.run_hash(max_iter, deltas, paths) : drv.run(max_iter, deltas);
        } catch (const Error &) {
            reached = drv.cur_iter;
            throw;
        }
        for (uint32_t p = 0; p < n_preds; ++p) {
            if (!drv.idb[p]) continue;
            DRel &f = drv.full[p];
            drv.drop_index(f);
            xlog_hip_rel *r;
            if (f.n == 0) {
                r = rel_new(ctx, 2, 0);
            } else if (f.owned) {
                r = rel_adopt(ctx, 2, f.n, f.k, nullptr, REL_CANONICAL);
                f.owned = false;
            } else {
                r = rel_new(ctx, 2, f.n);
                r->rows = f.n;
                copy_d2d(ctx, r->w[0], f.k, f.n);
            }
            r->flags = REL_CANONICAL;
            out[p] = r;
        }
        if (stats) stats->route = use_hash ? XLOG_HIP_ROUTE_HASH : XLOG_HIP_ROUTE_JOIN;
    }
    XH_CHECK_HIP(hipEventRecord(ctx->ev_b, ctx->stream));
    XH_CHECK_HIP(hipEventSynchronize(ctx->ev_b));
    float ms = 0.f;
    XH_CHECK_HIP(hipEventElapsedTime(&ms, ctx->ev_a, ctx->ev_b));
    ctx->last_delta_sizes = deltas;
    ctx->last_iterations = iterations;
    if (stats) {
        stats->iterations = iterations;
        stats->wall_ms = ms;
        if (stats->delta_sizes)
            for (uint64_t i = 0; i < stats->delta_cap && i < deltas.size(); ++i) stats->delta_sizes[i] = deltas[i];
        stats->delta_count = std::min<uint64_t>(deltas.size(), stats->delta_sizes ? stats->delta_cap : 0);
    }
}

// The fixpoint with its statistics: on failure too, the iterations and delta
// sizes reached are reported, and host_waits counts the device waits.
void run_fixpoint(Ctx *ctx, const int32_t *plan, uint32_t n_preds, const xlog_hip_rel *const *rels, xlog_hip_rel **out,
                  xlog_hip_fixpoint_stats *stats) {
    const uint64_t waits0 = ctx->host_waits;
    std::vector<uint64_t> deltas;
    uint64_t reached = 0;  // the iteration a failure happened in (0: set-up or seed), when the route knows it
    try {
        run_fixpoint_impl(ctx, plan, n_preds, rels, out, stats, deltas, reached);
    } catch (...) {
        if (stats) {
            // the iterations completed, or the one in progress when it failed: the reference's counter is
            // incremented at the top of each iteration (recursive.rs:619-620)
            stats->iterations = std::max<uint64_t>(deltas.empty() ? 0 : deltas.size() - 1, reached);
            if (stats->delta_sizes)
                for (uint64_t i = 0; i < stats->delta_cap && i < deltas.size(); ++i) stats->delta_sizes[i] = deltas[i];
            stats->delta_count = std::min<uint64_t>(deltas.size(), stats->delta_sizes ? stats->delta_cap : 0);
            stats->host_waits = ctx->host_waits - waits0;
        }
        throw;
    }
    if (stats) stats->host_waits = ctx->host_waits - waits0;
}

}  // namespace xh
