// Host-layer declarations shared by abi.hip (relation helpers, operators and
// the C ABI) and fixpoint.hip (the semi-naive fixpoint driver).
#pragma once

#include "internal.hpp"

#include <utility>
#include <vector>

namespace xh {

// Owns one pool block until it is released: an error unwinding past the owner
// gives the block back to the pool.
struct Owned {
    Ctx *ctx;
    uint64_t *p;
    explicit Owned(Ctx *c, uint64_t *q = nullptr) : ctx(c), p(q) {}
    Owned(const Owned &) = delete;
    Owned &operator=(const Owned &) = delete;
    ~Owned() {
        if (p) ctx->free(p);
    }
    void reset(uint64_t *q = nullptr) {
        if (p && p != q) ctx->free(p);
        p = q;
    }
    uint64_t *release() {
        uint64_t *q = p;
        p = nullptr;
        return q;
    }
};
uint64_t *alloc_keys(Ctx *ctx, uint64_t n);

// Bags of packed tuples, each an owned pool block (a rule body's head tuples,
// a join's output): what is still held is freed when an error unwinds past
// the owner.
struct Bags {
    Ctx *ctx;
    std::vector<std::pair<uint64_t *, uint64_t>> v;
    // per bag: 0, or (its rows grouped by their high word, in ascending order)
    // a bound on the number of groups
    std::vector<uint64_t> grouped;
    explicit Bags(Ctx *c) : ctx(c) {}
    Bags(Bags &&o) noexcept : ctx(o.ctx), v(std::move(o.v)), grouped(std::move(o.grouped)) {
        o.v.clear();
        o.grouped.clear();
    }
    Bags(const Bags &) = delete;
    Bags &operator=(const Bags &) = delete;
    ~Bags() { clear(); }
    void clear() {
        for (auto &b : v)
            if (b.first) ctx->free(b.first);
        v.clear();
        grouped.clear();
    }
    void add(Owned &o, uint64_t n, uint64_t groups = 0) {
        v.push_back({o.p, n});
        grouped.push_back(groups);
        o.release();
    }
    uint64_t rows() const {
        uint64_t t = 0;
        for (auto &b : v) t += b.second;
        return t;
    }
};
std::vector<Bags> bags_per_pred(Ctx *ctx, uint32_t n);

// Canonical (sorted, unique) copy of the packed keys of an arity<=2 relation,
// or the relation's own buffer when it is already canonical (owned = null).
struct Canon {
    Ctx *ctx = nullptr;
    const uint64_t *k = nullptr;
    uint64_t n = 0;
    uint64_t *owned = nullptr;
    ~Canon() { if (owned && ctx) ctx->free(owned); }
};

// Join index over one column of an arity<=2 relation: sorted (key, other)
// pairs, run index and payload (= other column, key order).
struct JoinIndex {
    RunIndex ix;
    Buf<uint32_t> payload;
    uint64_t n = 0;
};

// one device count read back (waits for the stream)
uint64_t read_count(Ctx *ctx, const uint64_t *d);
void copy_d2d(Ctx *ctx, uint64_t *dst, const uint64_t *src, uint64_t n);
// a relation adopting device word buffers (ownership moves to it)
xlog_hip_rel *rel_adopt(Ctx *ctx, uint32_t arity, uint64_t rows, uint64_t *w0, uint64_t *w1, uint32_t flags);
// (a, b) words -> (word h0, word h1) words of n packed pairs (h in {0, 1})
void project_pairs(Ctx *ctx, const uint64_t *in, uint64_t n, int h0, int h1, uint64_t *out);
// Sorted copy of n packed keys (keys_owned: the input buffer is consumed) by
// the digits [digit_lo, digit_hi); known_digits: the digits that may vary (0:
// from the histograms); whole (a sort of digits 4..7): set when the keys came
// out ordered by the whole key (the segment route).
uint64_t *sort_keys(Ctx *ctx, uint64_t *keys, uint64_t n, bool keys_owned, int digit_lo = 0, int digit_hi = 8,
                    uint32_t known_digits = 0, bool *whole = nullptr);
// Sorted unique copy of n keys into a new buffer *out, the count to *d_count (device).
void sort_unique_keys_async(Ctx *ctx, const uint64_t *keys, uint64_t n, uint64_t **out, uint64_t *d_count,
                            uint32_t known_digits = 0);
// Join index over column `col` of packed rows of `arity` <= 2 (payload_sorted:
// ascending payloads inside a run; unique_rows: duplicate rows dropped).
void build_join_index(Ctx *ctx, const uint64_t *keys, uint64_t n, uint32_t arity, int col, bool canonical,
                      JoinIndex &J, bool payload_sorted = false, bool unique_rows = false);
// The emit side of a join step whose count pass has run, and a whole join step
// (probe rows against J, two-column outputs oc, set semantics in pieces past
// the chunk size; max_rows, when non-zero, is the join-row limit; digits: the
// sort's known varying digits).
uint64_t join_emit(Ctx *ctx, ProbeJob &job, const int oc[4], uint64_t **out, uint64_t max_rows, uint32_t digits);
uint64_t join_step(Ctx *ctx, const uint64_t *probe, uint64_t n, int pcol, const JoinIndex &J, const int oc[4],
                   uint64_t **out, uint64_t max_rows = 0, uint32_t digits = 0);
// flags[i] = 1 when row i's (key word pcol, other word) pair is a row of the
// indexed relation (an index on its first column, payloads ascending per run)
void join_match2_flags(Ctx *ctx, const uint64_t *probe, uint64_t n, int pcol, const RunIndex &ix,
                       const uint32_t *payload, uint8_t *flags);
// flags[i] = 1 when mask row i, (u, v) (or (v, u) with mask_swap), has a w in both
// the run of u in P and the run of v in Q (payloads ascending per run)
void wcoj_triangle_flags(Ctx *ctx, const uint64_t *mask, uint64_t n, int mask_swap, const RunIndex &P,
                         const uint32_t *p_payload, const RunIndex &Q, const uint32_t *q_payload, uint8_t *flags);
// *mx = max(*mx, the largest of both 32-bit halves of n packed words)
void max_u32_of_packed(Ctx *ctx, const uint64_t *k, uint64_t n, unsigned int *mx);
// XLOG_HIP_TRACE=1: progress lines on stderr
bool trace_on();
// a positive integer from the environment, or dflt
uint64_t env_u64(const char *name, uint64_t dflt);
// device bytes an operation may still take (free memory within the budget)
uint64_t device_room(Ctx *ctx);
// the semi-naive fixpoint (fixpoint.hip), statistics included
void run_fixpoint(Ctx *ctx, const int32_t *plan, uint32_t n_preds, const xlog_hip_rel *const *rels, xlog_hip_rel **out,
                  xlog_hip_fixpoint_stats *stats);

}  // namespace xh
