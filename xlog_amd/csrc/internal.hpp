// Internal declarations shared by the HIP translation units of libxlog_hip.
// Everything here is gfx950 (wave64) code; the public surface is the C ABI
// declared in include/xlog_hip.h.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstddef>
#include <cstring>
#include <string>
#include <vector>
#include <map>
#include <mutex>

#include "../../include/xlog_hip.h"

namespace xh {

constexpr int WAVE = 64;

// Block-strided copy of n items, st(i, ld(i)) for i in [0, n), with BATCH loads
// in flight per thread: a plain strided loop waits for each load before its
// store, so staging a tile costs one memory latency per item a thread copies.
// Loads past n read item n - 1 (in bounds, results dropped).  Every thread of
// the block calls it with the same n.
template <int BLOCK, int BATCH, class Load, class Store>
__device__ __forceinline__ void batched_copy(uint32_t n, int tid, Load ld, Store st) {
    for (uint32_t base = 0; base < n; base += (uint32_t)(BLOCK * BATCH)) {
        decltype(ld(0u)) v[BATCH];
#pragma unroll
        for (int q = 0; q < BATCH; ++q) {
            const uint32_t i = base + (uint32_t)(q * BLOCK + tid);
            v[q] = ld(i < n ? i : n - 1);
        }
#pragma unroll
        for (int q = 0; q < BATCH; ++q) {
            const uint32_t i = base + (uint32_t)(q * BLOCK + tid);
            if (i < n) st(i, v[q]);
        }
    }
}

// ---------------------------------------------------------------------------
// error plumbing: every entry point returns a status and leaves a message in
// a thread-local buffer readable through xlog_hip_last_error().
// ---------------------------------------------------------------------------
void set_error(const std::string &msg);
struct Error {
    xlog_hip_status code;
    std::string msg;
};

#define XH_CHECK_HIP(expr)                                                          \
    do {                                                                            \
        hipError_t _e = (expr);                                                     \
        if (_e != hipSuccess)                                                       \
            throw ::xh::Error{XLOG_HIP_DEVICE_ERROR,                                \
                              std::string(#expr) + ": " + hipGetErrorString(_e)};   \
    } while (0)

#define XH_REQUIRE(cond, code, msg)                                                 \
    do {                                                                            \
        if (!(cond)) throw ::xh::Error{code, msg};                                  \
    } while (0)

// ---------------------------------------------------------------------------
// stream-ordered caching allocator.  All work of a context runs on its one
// stream, so a block freed by one operation can be handed to the next one
// without a synchronisation: the stream orders the reuse after the last use.
// ---------------------------------------------------------------------------
class Pool {
  public:
    explicit Pool(int device) : device_(device) {}
    int device() const { return device_; }
    ~Pool();
    void *alloc(size_t bytes);
    void free(void *p);
    void trim();  // return cached blocks to the driver
    size_t bytes_in_use() const { return in_use_; }
    size_t bytes_cached() const { return cached_; }
    size_t peak_in_use() const { return peak_; }
    // Device memory budget (0: none): an allocation that would take the live
    // bytes past it fails with XLOG_HIP_OOM, and cached blocks are returned to
    // the driver before the pool's footprint (live + cached) would pass it.
    void set_budget(size_t bytes) { budget_ = bytes; }
    size_t budget() const { return budget_; }
    // bytes the budget still allows (SIZE_MAX without one)
    size_t headroom() const { return budget_ ? (budget_ > in_use_ ? budget_ - in_use_ : 0) : SIZE_MAX; }

  private:
    static size_t round_up(size_t b);
    int device_;
    std::multimap<size_t, void *> free_;  // size class -> block
    std::map<void *, size_t> live_;
    size_t in_use_ = 0, cached_ = 0, peak_ = 0, budget_ = 0;
};

// RAII scratch buffer from the context pool
struct Ctx;
template <typename T>
struct Buf {
    Ctx *ctx = nullptr;
    T *p = nullptr;
    size_t n = 0;
    Buf() = default;
    Buf(Ctx *c, size_t count);
    Buf(const Buf &) = delete;
    Buf &operator=(const Buf &) = delete;
    Buf(Buf &&o) noexcept : ctx(o.ctx), p(o.p), n(o.n) { o.p = nullptr; o.n = 0; }
    Buf &operator=(Buf &&o) noexcept;
    ~Buf();
    T *release() { T *q = p; p = nullptr; n = 0; return q; }
};

// ---------------------------------------------------------------------------
// context: one device, one stream, the pool and the small persistent device
// state used by the single-pass (decoupled look-back) kernels.
// ---------------------------------------------------------------------------
struct Ctx {
    int device = 0;
    int num_cus = 0;
    hipStream_t stream = nullptr;
    Pool *pool = nullptr;
    // pinned host staging for scalar read-backs
    static constexpr size_t HOST_STAGE_U64 = 2048;  // 16 KB: scalars, counts, the sort's 8 x 256 histogram
    uint64_t *host_scalars = nullptr;  // HOST_STAGE_U64 entries
    // device scratch: ticket counters for tile ordering (monotone, never reset)
    unsigned long long *tickets = nullptr;  // 16 counters
    unsigned long long ticket_base[16] = {0};
    hipEvent_t ev_a = nullptr, ev_b = nullptr;
    hipEvent_t ev_sync = nullptr;  // no timing; sync() polls it
    hipEvent_t ev_read = nullptr;  // no timing; marks a read-back that later launches may overtake
    // statistics of the last fixpoint / op (host side)
    std::vector<uint64_t> last_delta_sizes;
    uint64_t last_iterations = 0;
    float last_kernel_ms = 0.f;

    // per-kernel-kind timing with HIP events on `stream` (off unless enabled)
    struct ProfRec {
        int kind;
        hipEvent_t a, b;
        double bytes;
        int work_slot;         // device work counter of the launch (-1: none)
        double bytes_per_work; // algorithmic bytes per counted work unit
    };
    bool profiling = false;
    std::vector<ProfRec> prof_pending;
    std::vector<hipEvent_t> prof_events;
    double prof_ms[XLOG_HIP_KERNEL_KINDS] = {0};
    double prof_bytes[XLOG_HIP_KERNEL_KINDS] = {0};
    uint64_t prof_launches[XLOG_HIP_KERNEL_KINDS] = {0};
    hipEvent_t prof_event() {
        if (!prof_events.empty()) {
            hipEvent_t e = prof_events.back();
            prof_events.pop_back();
            return e;
        }
        hipEvent_t e;
        XH_CHECK_HIP(hipEventCreate(&e));
        return e;
    }
    void prof_resolve();  // synchronises, folds pending records into the totals
    // device counters that profiled launches add their work units to; read
    // back and cleared by prof_resolve
    static constexpr int PROF_WORK_SLOTS = 16384;
    // each slot is PROF_WORK_SPREAD counters: a launch's blocks add to counter
    // (block id mod PROF_WORK_SPREAD) so that thousands of blocks do not
    // serialise on one address
    static constexpr int PROF_WORK_SPREAD = 64;
    unsigned long long *prof_work = nullptr;
    int prof_work_next = 0;

    void *alloc(size_t bytes) { return pool->alloc(bytes); }
    void free(void *p) { pool->free(p); }
    // reserve `count` consecutive ticket values on counter `slot`; returns the
    // base that the kernel subtracts from its atomicAdd result.
    unsigned long long take_tickets(int slot, unsigned long long count) {
        unsigned long long b = ticket_base[slot];
        ticket_base[slot] += count;
        return b;
    }
    // Waits for the stream by polling an event: a read-back is followed by a
    // launch that depends on the value, and a blocking wait's wake-up adds tens
    // of microseconds of idle device per read-back (the host core spins instead).
    uint64_t host_waits = 0;  // waits for the device (read-backs, synchronisations)
    void wait_event(hipEvent_t ev) {
        ++host_waits;
        hipError_t e;
        while ((e = hipEventQuery(ev)) == hipErrorNotReady) {
        }
        XH_CHECK_HIP(e);
    }
    void sync() {
        XH_CHECK_HIP(hipEventRecord(ev_sync, stream));
        wait_event(ev_sync);
    }
    // D2H of a few u64 scalars through pinned memory (synchronises)
    void read_scalars(const void *dev, size_t count_u64);
};

// Brackets one launch with events when profiling is on.
struct Prof {
    Ctx *ctx;
    Ctx::ProfRec rec;
    bool on;
    Prof(Ctx *c, int kind, double bytes) : ctx(c), on(c->profiling) {
        if (!on) return;
        rec.kind = kind;
        rec.bytes = bytes;
        rec.work_slot = -1;
        rec.bytes_per_work = 0.0;
        rec.a = c->prof_event();
        rec.b = c->prof_event();
        XH_CHECK_HIP(hipEventRecord(rec.a, c->stream));
    }
    // A zeroed device counter for the launch to add work units to (each worth
    // bytes_per_unit algorithmic bytes), or null when not profiling.
    unsigned long long *work(double bytes_per_unit);
    ~Prof() {
        if (!on) return;
        (void)hipEventRecord(rec.b, ctx->stream);
        ctx->prof_pending.push_back(rec);
    }
};

template <typename T>
Buf<T>::Buf(Ctx *c, size_t count) : ctx(c), n(count) {
    p = count ? static_cast<T *>(c->alloc(count * sizeof(T))) : nullptr;
}
template <typename T>
Buf<T> &Buf<T>::operator=(Buf &&o) noexcept {
    if (this != &o) {
        if (p && ctx) ctx->free(p);
        ctx = o.ctx; p = o.p; n = o.n;
        o.p = nullptr; o.n = 0;
    }
    return *this;
}
template <typename T>
Buf<T>::~Buf() {
    if (p && ctx) ctx->free(p);
}

}  // namespace xh

// ---------------------------------------------------------------------------
// relation handle (the CudaBuffer counterpart).  Rows are stored as packed
// u64 words, row-major within a word, word-major across words:
//   arity 1:    w[0][i] = c0
//   arity 2k:   w[j][i] = (c_{2j} << 32) | c_{2j+1}          (j < k)
//   arity 2k+1: as 2k + 2 with the last column zero
// e.g. arity 3: w[0][i] = (c0 << 32) | c1, w[1][i] = c2 << 32.  Arity is 1..8
// (four words).  Unsigned u64 order over (w[0], w[1], ...) is the
// lexicographic unsigned column order, and equal words are bytewise-equal rows.
// ---------------------------------------------------------------------------
namespace xh {
constexpr uint32_t MAX_ARITY = 8;
constexpr int MAX_WORDS = 4;
inline int words_for(uint32_t arity) { return arity <= 2 ? 1 : (int)((arity + 1) / 2); }
}  // namespace xh
struct xlog_hip_rel {
    xh::Ctx *ctx = nullptr;
    uint32_t arity = 0;
    uint64_t rows = 0;
    uint64_t cap = 0;
    uint64_t *w[xh::MAX_WORDS] = {nullptr, nullptr, nullptr, nullptr};
    uint32_t flags = 0;  // XLOG_HIP_REL_CANONICAL when sorted by all columns and unique
    int nwords() const { return xh::words_for(arity); }
};

namespace xh {

constexpr uint32_t REL_CANONICAL = 1u;

xlog_hip_rel *rel_new(Ctx *ctx, uint32_t arity, uint64_t cap);
void rel_free(xlog_hip_rel *r);

// ---------------------------------------------------------------------------
// device algorithm entry points (host wrappers around the kernels); all
// stream-ordered on ctx->stream.
// ---------------------------------------------------------------------------

// LSD radix sort of u64 keys with an optional u32 payload, stable, over the
// 8-bit digits [digit_lo, digit_hi) (0..8 = the whole key; 4..8 = the high
// word only).  On return *keys (and *vals) point at whichever of the two
// buffers holds the result; the other is scratch.  The pass of the lowest
// digit always runs (it is queued before the histograms are read back); every
// higher digit that is constant over the input is skipped.  A keys-only sort
// of the whole key over at least 2^22 keys instead waits for the histograms,
// and when they predict that the high word leaves runs of a few keys, runs
// the high word's passes and one sort_short_runs pass (the low word's passes
// only if some run exceeds 256 keys).  Returns the number of passes executed.
// With `src` (keys only) the first pass reads src and both buffers are
// scratch, so an input that must not be modified is never copied first.
// With known_digits (a bitmask of digits that may vary, e.g. from the value
// domain) the passes are exactly those digits of [digit_lo, digit_hi) and the
// histograms are not read back (a known digit that turns out constant costs a
// stable copy).
// Keys sorted by their high word to keys sorted in full, out of place: every
// run of equal high word is sorted by the low word.  A run longer than 256
// keys sets *d_long (device) and leaves the output incomplete; the caller then
// sorts the input in full instead.
void sort_short_runs(Ctx *ctx, const uint64_t *in, uint64_t n, uint64_t *out, uint64_t *d_long);
// With `uq` (a keys-only sort of the whole key) the high-word route, when
// taken, also deduplicates: *keys then holds the uq->count unique keys and
// uq->done is set; otherwise *keys holds all n keys, sorted.
struct SortUnique {
    bool done = false;
    uint64_t count = 0;
};
// XLOG_HIP_SORT_TICKETS=1 (read at each sort): the radix pass and the
// short-run unique order their tiles by an atomic start ticket instead of the
// workgroup index, so that their look-back does not rest on workgroups
// starting in index order (slower: one device-wide atomic per tile).
bool sort_tickets();
// With `whole` (a keys-only sort of the high word, digits 4..7, of at least
// 2^22 keys) the sort may order the keys by the whole key instead, through the
// segment route; *whole tells whether it did.
int radix_sort_u64(Ctx *ctx, uint64_t **keys, uint64_t **keys_alt, uint32_t **vals, uint32_t **vals_alt,
                   uint64_t n, int digit_lo = 0, int digit_hi = 8, const uint64_t *src = nullptr,
                   uint32_t known_digits = 0, SortUnique *uq = nullptr, bool *whole = nullptr);
// A keys-only sort of a queued iteration: the key count on the device
// (*d_n <= n_bound, the bound the launches are sized for), exactly the digit
// passes of known_digits (no read-back), and the stop flag (a raised flag:
// nothing is done).  Returns the number of passes: *keys and *keys_alt are
// swapped once per pass, as in radix_sort_u64.
// Grid of a launch over `tiles` tiles whose real count is on the device: at
// most a few blocks per CU, which stride over (or take tickets for) the tiles.
// Persistent launches that take tickets use counter PERSIST_TICKET_SLOT (the
// radix pass PERSIST_TICKET_SLOT + 1) with base 0, and the counter two slots
// further on to count the blocks that are done.  Only the first `parts`
// blocks (at most one per tile that holds rows) take tickets; the last of
// them to finish zeroes both counters (persist_done), so each launch finds
// them at zero.
constexpr int PERSIST_TICKET_SLOT = 8;
__device__ __forceinline__ void persist_done(unsigned long long *ticket, uint64_t parts) {
    if (atomicAdd(ticket + 2, 1ull) == (unsigned long long)(parts - 1)) {
        ticket[0] = 0ull;
        ticket[2] = 0ull;
    }
}
inline unsigned persistent_grid(const Ctx *ctx, uint64_t tiles, uint32_t per_cu = 8) {
    const uint64_t cap = (uint64_t)ctx->num_cus * per_cu;
    return (unsigned)(tiles < cap ? (tiles ? tiles : 1) : cap);
}
// Profiling of a launch sized by bounds: adds wa * min(*d_a, a) + wb *
// min(*d_b, b) (a device count given as null counts its bound) to the
// launch's work counter, unless *stop is raised or *skip is zero; nothing
// without a counter.
void add_work_rows(Ctx *ctx, unsigned long long *work, const uint64_t *d_a, uint64_t a, uint32_t wa, const uint64_t *d_b,
                   uint64_t b, uint32_t wb, const uint64_t *skip, const uint32_t *stop);
// Sort of keys grouped by their high word (every key of a high word in one
// run, the runs in ascending order) in a queued iteration: one short-run pass
// (each run ordered by its low word) from keys to keys_alt; when a run is
// longer than 256 keys, the digit passes of known_digits run instead (decided
// on the device, no read-back).  The result is in the returned buffer,
// keys_alt; keys is overwritten.  scratch: two device words.
uint64_t *sort_grouped_dev(Ctx *ctx, uint64_t *keys, uint64_t *keys_alt, uint64_t n_bound, const uint64_t *d_n,
                           uint32_t known_digits, const uint32_t *stop, uint64_t *scratch);
int radix_sort_dev(Ctx *ctx, uint64_t **keys, uint64_t **keys_alt, uint64_t n_bound, const uint64_t *d_n,
                   uint32_t known_digits, const uint32_t *stop);
// sort_short_runs fused with the adjacent-compare unique: the unique keys in
// order to `out`, their count to *d_count (device); a run longer than 256
// keys sets *d_long and the output is then incomplete.  Its tiles take their
// order from the workgroup index, like the radix pass, unless sort_tickets().
void sort_short_runs_unique(Ctx *ctx, const uint64_t *in, uint64_t n, uint64_t *out, uint64_t *d_count,
                            uint64_t *d_long);
// Segment route of a large full-key sort: `in` holds n keys ordered by their
// top 16 bits; a segment is the keys of 2^gshift consecutive top-16-bit values
// (gshift in [0, 8]), and every segment is sorted by the rest of the key on
// chip, one block per segment.  With d_count the unique keys go to `out` in
// order and their count to *d_count (device); without it all n keys go to
// `out`, sorted.  A segment of more than SORT_SEGMENT_MAX keys, or more than
// 256 keys that share bits 36 + gshift .. 63 and are not all equal, sets
// *d_long and the output is then incomplete.
constexpr uint64_t SORT_SEGMENT_MAX = 5120;
void sort_top_segments(Ctx *ctx, const uint64_t *in, uint64_t n, uint64_t *out, uint64_t *d_count, uint64_t *d_long,
                       int gshift);

// Stream compaction family (single pass, decoupled look-back).  Each writes
// the selected keys in input order to `out` and the count to *d_count
// (device) ; returns nothing, the caller reads the count when it needs it.
// Where a d_n argument is taken and set, the input's row count is *d_n on the
// device and n only the bound the launch is sized for.
//   unique:      keep k[i] if i == 0 or k[i] != k[i-1]                 (sorted input)
//   unique_diff: keep k[i] if unique and k[i] not in sorted b[0..nb)
//   diff:        keep k[i] if k[i] not in sorted b[0..nb)
void select_unique(Ctx *ctx, const uint64_t *k, uint64_t n, uint64_t *out, uint64_t *d_count,
                   const uint64_t *d_n = nullptr);
//   unique_low:  unique, and the low word of each selected key to low[]
void select_unique_low(Ctx *ctx, const uint64_t *k, uint64_t n, uint64_t *out, uint32_t *low, uint64_t *d_count);
void select_unique_diff(Ctx *ctx, const uint64_t *k, uint64_t n, const uint64_t *b, uint64_t nb,
                        uint64_t *out, uint64_t *d_count);
// The same with the row counts of k and b on the device (d_n, d_nb; n and nb
// are then the bounds the launches are sized for; b must be a valid pointer)
// and the stop flag of a queued iteration (a raised flag: nothing is done).
void select_unique_diff_dev(Ctx *ctx, const uint64_t *k, uint64_t n, const uint64_t *d_n, const uint64_t *b,
                            uint64_t nb, const uint64_t *d_nb, uint64_t *out, uint64_t *d_count, const uint32_t *stop);
// The same against two sorted arrays at once (not in b and not in b2; b2's
// count on the device when d_nb2 is set, nb2 its bound).
void select_unique_diff2_dev(Ctx *ctx, const uint64_t *k, uint64_t n, const uint64_t *d_n, const uint64_t *b,
                             uint64_t nb, const uint64_t *d_nb, const uint64_t *b2, uint64_t nb2, const uint64_t *d_nb2,
                             uint64_t *out, uint64_t *d_count, const uint32_t *stop);
void select_flags(Ctx *ctx, const uint64_t *k, const uint8_t *flags, uint64_t n, uint64_t *out,
                  uint64_t *d_count);
//   not_value:   keep k[i] if k[i] != v
void select_not_value(Ctx *ctx, const uint64_t *k, uint64_t n, uint64_t v, uint64_t *out, uint64_t *d_count,
                      const uint64_t *d_n = nullptr, const uint32_t *stop = nullptr);
// Sorted unique difference of grouped candidates over a domain of at most
// 2^17 values (every low word below `domain`): the candidates (count
// *d_cand <= cand_bound) come in groups of one high word, listed by
// select_runs (*d_nruns <= runs_bound); R is a sorted base run of nbase rows
// and a sorted recent run (*d_nrecent <= recent_bound).  Each group's values
// that are not in R go, ascending, to slots from the group's first position,
// the rest of its positions get `hole`; compacting the slots
// (select_not_value) gives the sorted new rows.  With rin (R as a bit
// matrix, rows_to_bits) R's rows come from it, and rout receives the rows of
// the groups with their values added (R after the iteration; the caller
// copies the other rows).
void group_bitmap_diff_dev(Ctx *ctx, const uint64_t *cand, uint64_t cand_bound, const uint64_t *d_cand,
                           const uint32_t *run_key, const uint64_t *run_start, uint64_t runs_bound,
                           const uint64_t *d_nruns, const uint64_t *base, uint64_t nbase, const uint64_t *recent,
                           uint64_t recent_bound, const uint64_t *d_nrecent, uint32_t domain, uint64_t hole,
                           uint64_t *slots, const uint64_t *rin, uint64_t *rout, const uint32_t *stop);
// R (a sorted base run of nbase rows and a sorted recent run of nrec rows,
// every value below `domain` <= 2^17) as a bit matrix: domain rows of
// ceil(domain / 64) u64 words (bitmap_emit's layout).
void rows_to_bits(Ctx *ctx, const uint64_t *base, uint64_t nbase, const uint64_t *recent, uint64_t nrec,
                  uint32_t domain, uint64_t *bits);
// Rows run_key[0 .. *d_n) (at most bound) of a bit matrix over `domain`
// values copied from src to dst (nothing once *stop is set).
void copy_group_rows(Ctx *ctx, const uint32_t *run_key, const uint64_t *d_n, uint64_t bound, uint32_t domain,
                     const uint64_t *src, uint64_t *dst, const uint32_t *stop);
// The bits of packed rows (x << 32) | z, rows[0 .. *d_n) (at most bound), in a
// bit matrix of `words` u64 words per row: set (atomic OR), or, with clear,
// every word that holds one of them zeroed (nothing once *stop is set).
void rows_bits(Ctx *ctx, const uint64_t *rows, const uint64_t *d_n, uint64_t bound, uint32_t words, uint64_t *bits,
               bool clear, const uint32_t *stop);

// In-place exclusive scan of u32 values (prefixes wrap modulo 2^32); the
// exact u64 sum goes to *d_total (device).  One pass, decoupled look-back.
void scan_u32_inplace(Ctx *ctx, uint32_t *a, uint64_t n, unsigned long long *d_total);
// The same scan with its scratch (ticket, total, look-back status) in a
// file-scope device array instead of pool memory: no device allocation.  At
// most SCAN_NOALLOC_MAX values; the total is read back (synchronises).
// scan_noalloc_init looks the array's address up on `device` (current).
constexpr uint64_t SCAN_NOALLOC_MAX = 1ull << 32;
void scan_noalloc_init(int device);
void scan_u32_inplace_noalloc(Ctx *ctx, uint32_t *a, uint64_t n, uint64_t *total);

// Merge of two sorted arrays (stable, a before b on ties) into out[na+nb].
void merge_sorted(Ctx *ctx, const uint64_t *a, uint64_t na, const uint64_t *b, uint64_t nb, uint64_t *out);
// The same with device row counts (d_na, d_nb; na and nb are the bounds), a
// stop flag and a skip word: nothing is written when *stop is raised or
// *skip is zero.
void merge_sorted_dev(Ctx *ctx, const uint64_t *a, uint64_t na, const uint64_t *d_na, const uint64_t *b, uint64_t nb,
                      const uint64_t *d_nb, uint64_t *out, const uint64_t *skip, const uint32_t *stop);

// Sorted-run index over the high word of sorted packed keys (join build):
// an open-addressing hash table of 16-byte slots mapping key -> (run start,
// run length) in the sorted keys.
struct RunIndex {
    Buf<unsigned long long> table;  // per slot: (key << 32) | run length (0 = empty), run start
    uint64_t nruns = 0;
    uint64_t table_mask = 0;
};
void build_run_index(Ctx *ctx, const uint64_t *sorted_keys, uint64_t n, RunIndex &ix);
// The same in two steps around one read-back: the runs of sorted_keys[0, n)
// with n = *d_n when d_n is set (n_bound sizes the buffers), run count to
// *d_nruns; then the table, once the run count and n are known.
struct RunScratch {
    Buf<uint32_t> run_key;
    Buf<uint64_t> run_start;
};
void build_run_index_async(Ctx *ctx, const uint64_t *sorted_keys, uint64_t n_bound, const uint64_t *d_n,
                           RunScratch &rs, uint64_t *d_nruns);
void build_run_index_finish(Ctx *ctx, RunScratch &rs, uint64_t nruns, uint64_t n, RunIndex &ix);
// The table of a run index whose runs are on the device (select_runs with a
// device row count: *d_nruns runs, at most runs_bound, over *d_n sorted keys):
// ix.table holds ix.table_mask + 1 >= 2 * runs_bound slots and is cleared and
// filled here, with no read-back; a raised stop leaves it cleared.
void run_index_insert_dev(Ctx *ctx, const uint32_t *run_key, const uint64_t *run_start, const uint64_t *d_nruns,
                          uint64_t runs_bound, const uint64_t *d_n, RunIndex &ix, const uint32_t *stop);
// Merge-path lookup of the sort-merge join: for every row of l (sorted by the
// key word pcol), the start and length of its run among the nr runs of
// (run_key, run_start[0..nr]) (sorted, distinct keys); length 0 without one.
void smj_lookup(Ctx *ctx, const uint64_t *l, uint64_t nl, int pcol, const uint32_t *run_key, const uint64_t *run_start,
                uint64_t nr, uint64_t *start, uint32_t *cnt);

// Probe: for every packed probe row p[i], key = column `pcol` of the row
// (0 = high word, 1 = low word); each match emits
//   out = (sel(p, oc0) << 32) | sel(p, oc1)
// where sel picks among (p.c0, p.c1, build.key, build.payload) by index 0..3.
// Two launches: count (per-tile totals with look-back) and emit.  Returns the
// number of output rows (one read-back).
uint64_t join_probe_project(Ctx *ctx, const uint64_t *probe, uint64_t n, int pcol, const RunIndex &ix,
                            const uint32_t *payload, int oc0, int oc1, uint64_t **out);

// Probe in pieces: a count pass over all probe tiles (tile offsets on the
// device, total read back), then emits of tile ranges.  Tile t covers probe
// rows [t * 256 * items, (t + 1) * 256 * items).
struct ProbeJob {
    const uint64_t *probe = nullptr;
    uint64_t n = 0;
    int pcol = 0;
    const RunIndex *ix = nullptr;
    const uint32_t *payload = nullptr;
    // Optional row groups, for 2-column outputs: gsel[i] = -1 plain row, -2
    // a row with no output, g >= 0 a row whose outputs are the finished words
    // gsrc[gseg[2g] .. gseg[2g] + gseg[2g + 1]) instead of its matches.
    const int32_t *gsel = nullptr;
    const uint64_t *gseg = nullptr;  // (start, count) per group
    const uint64_t *gsrc = nullptr;
    // Optional precomputed lookups (sort-merge join): run start and length
    // per probe row, used instead of the index's hash table.
    const uint64_t *pre_start = nullptr;
    const uint32_t *pre_cnt = nullptr;
    // probe_prepare records the count pass's lookups (12 B per probe row) and
    // points pre_start / pre_cnt at them for the emit
    bool record_lookups = true;
    Buf<uint64_t> rec_start;
    Buf<uint32_t> rec_cnt;
    Buf<uint64_t> toff;  // exclusive prefix of per-tile output counts; toff[tiles] = total
    uint64_t tiles = 0, total = 0;
    int items = 16;      // probe rows per thread (set by probe_prepare); a tile is 256 * items rows
};
uint64_t probe_prepare(Ctx *ctx, ProbeJob &job);
// The count pass for a probe whose row count is on the device (*d_n <= n_bound),
// with no read-back; the total lands at job.toff.p[job.tiles].  probe_finish
// completes the job once the host has read the row count and the total.
// In a queued iteration, stop is the queue's stop flag and stop_code (when
// non-zero) the code the count raises when *d_n is past n_bound.
void probe_prepare_deferred(Ctx *ctx, ProbeJob &job, uint64_t n_bound, const uint64_t *d_n,
                            uint32_t *stop = nullptr, uint32_t stop_code = 0);
// The emit of a deferred probe inside a queued iteration: the probe rows'
// count on the device (d_n, at most job.n), two-column outputs (oc) written
// to out + *d_out_base (d_out_base may be null), nothing when *stop is raised.
// The caller has checked that the total fits the output.
// With a filter (two-column outputs of ids below 64 * words): an output
// already in R (bit set in rbits, a bit matrix of `words` u64 words per row;
// may be null) or already taken (bit set in seen, which the emit sets) is
// dropped, the others are appended in no set order at out[*count] (*count
// advanced; positions at or past cap are counted and not written).
struct EmitFilter {
    const uint64_t *rbits;
    uint64_t *seen;
    uint64_t *count;
    uint64_t cap;
    uint32_t words;
};
void probe_emit_dev(Ctx *ctx, const ProbeJob &job, const uint64_t *d_n, const int oc[4], uint64_t *out,
                    const uint64_t *d_out_base, uint32_t *stop, const EmitFilter *filter = nullptr);
void probe_finish(ProbeJob &job, uint64_t n, uint64_t total);
// The count pass alone, lookups recorded, no scan and no read-back; with gsel
// set and gseg null the group heads count zero until probe_group_fixup gives
// each head (row hpos[g]) its group's finished words gseg[2g], gseg[2g + 1].
// probe_scan_async then leaves the total at job.toff.p[job.tiles].
void probe_count_only(Ctx *ctx, ProbeJob &job);
void probe_group_fixup(Ctx *ctx, ProbeJob &job, const uint64_t *hpos, const uint64_t *gseg, uint64_t nh);
void probe_scan_async(Ctx *ctx, ProbeJob &job);
std::vector<uint64_t> probe_tile_offsets(Ctx *ctx, const ProbeJob &job);
// writes the `rows` outputs of tiles [t0, t1) to out0 / out1 starting at index 0
void probe_emit_range(Ctx *ctx, const ProbeJob &job, uint64_t t0, uint64_t t1, uint64_t rows, int out_arity,
                      const int oc[4], uint64_t *out0, uint64_t *out1);

// Device hash set of packed u64 tuples (hash_set.hip): open addressing,
// linear probing, the all-ones key kept as a flag.  flags[0] = all-ones key
// present, flags[1] = overflow of the last insert pass, flags[2] = tuples
// appended by the last novel-insert pass (the host zeroes [1] and [2]).
struct HashSet {
    Buf<uint64_t> slots;
    Buf<uint64_t> flags;
    uint64_t cap = 0;   // slots, a power of two
    int bits = 0;
    uint64_t size = 0;  // tuples held (host bookkeeping)
};
void hs_init(Ctx *ctx, HashSet &h, uint64_t min_cap);
// inserts keys without novelty bookkeeping (flags[1] set on a full table);
// the all-ones key sets flags[0]
void hs_insert_all(Ctx *ctx, HashSet &h, const uint64_t *keys, uint64_t n);
// rehash into a table of at least min_cap slots
void hs_grow(Ctx *ctx, HashSet &h, uint64_t min_cap);
// One sparse factorized delta step: for every delta row (carry, key) and
// every run entry of key in the index (values in payload), insert
// head(carry, value) (carry in the high word when out_carry_hi); the inserted
// tuples are appended to out at flags[2].  Once the appended count reaches
// `limit` (or the table is full) flags[1] is set and the pass stops early; out
// needs limit + HS_APPEND_SLACK entries.
void hs_join_insert(Ctx *ctx, HashSet &h, const uint64_t *delta, uint64_t n, int key_hi, int out_carry_hi,
                    const RunIndex &ix, const uint32_t *payload, uint64_t *out, uint64_t limit);
// One step of a queue of fixpoint steps launched with no read-back between
// them: the step's row count is on the device (d_n; the host's n is a bound),
// stop[0 .. nprior) are the overflow flags of the earlier steps (any one set:
// the launch does nothing) and prior[t * stride] for t < nprior the tuples
// this head appended in them.  `room` bounds the appends of all the steps
// together (the set stays at most half full): the launch's limit is cut to
// room minus the earlier steps' appends.
struct QueuedStep {
    const uint64_t *d_n = nullptr;
    const unsigned long long *stop = nullptr;
    const unsigned long long *prior = nullptr;
    int nprior = 0;
    int stride = 0;
    uint64_t room = ~0ull;
};
// inserts keys[0..n) and appends the novel ones (same protocol); optionally
// the keys' words exchanged (swap), the appended count and overflow flag
// elsewhere than the set's flags, and a queued step
void hs_insert_novel(Ctx *ctx, HashSet &h, const uint64_t *keys, uint64_t n, uint64_t *out, uint64_t limit,
                     int swap = 0, unsigned long long *count = nullptr, unsigned long long *overflow = nullptr,
                     const QueuedStep *q = nullptr);
// One step of a path-shaped rule body of two or three atoms, same protocol:
// every delta row, read as the path values (xa, xb) of the delta atom (the
// high then low word, swapped when delta_swap), is expanded through hop 1 (the
// run of xa or xb: values v1) and, when h2.table is set, each v1 through hop
// 2 (the run of xa, xb or v1: values v2); the head tuple (value out0, value
// out1) over the selectors 0 = xa, 1 = xb, 2 = v1, 3 = v2 is inserted.
struct PathHop {
    const unsigned long long *table = nullptr;  // run index slots (join.hip's build)
    uint64_t mask = 0;
    int bits = 0;
    const uint32_t *payload = nullptr;
};
struct PathInsertArgs {
    const uint64_t *delta = nullptr;
    uint64_t n = 0;  // delta rows (a bound in a queued step)
    QueuedStep q;    // optional: a queued step
    int delta_swap = 0;
    PathHop h1, h2;
    int key1 = 0;  // 0: xa, 1: xb
    int key2 = 0;  // 0: xa, 1: xb, 2: v1
    int out0 = 0, out1 = 0;
};
void hs_path_insert(Ctx *ctx, HashSet &h, const PathInsertArgs &a, uint64_t *out, uint64_t limit,
                    unsigned long long *count = nullptr, unsigned long long *overflow = nullptr);
// every tuple of the set, unordered, into out (h.size entries); returns the count
uint64_t hs_collect(Ctx *ctx, const HashSet &h, uint64_t *out);
// appends past `limit`: one 64-tuple chunk per wave of the insert grid
constexpr uint64_t HS_APPEND_SLACK = 1ull << 21;

// Nested-loop inner join of packed arity-1/2 relations on one key column,
// output (left columns ++ right columns) in left-row-major, right-row order.
// Returns the row count; out1 is set when the output arity exceeds 2.
uint64_t nested_loop_join(Ctx *ctx, const uint64_t *l, uint64_t nl, int la, int lk, const uint64_t *r, uint64_t nr,
                          int ra, int rk, uint64_t **out0, uint64_t **out1);

// One factorized TC delta step over a dense domain (ids < domain): the set
// {(x, z) : (x, y) in delta, (y, z) in edge, (x, z) not in full} as sorted
// unique packed (x << 32) | z rows.  delta and full are given as packed rows
// with the x column in the high (x_hi = 1) or low word; edge is sorted unique
// (y << 32) | z.  Returns the row count.
uint64_t fj_delta_step(Ctx *ctx, const uint64_t *delta, uint64_t nd, int delta_x_hi, const uint64_t *edge,
                       uint64_t ne, const uint64_t *full, uint64_t nf, int full_x_hi, uint32_t domain,
                       uint64_t **out);

// CSR of sorted unique packed (src << 32) | dst rows with ids < nv
// (row_ptr: nv + 1 entries, adj: m entries).
void pairs_csr(Ctx *ctx, const uint64_t *pairs, uint64_t m, uint32_t nv, uint64_t *row_ptr, uint32_t *adj);
// Set bits of an nv x words bitmap as sorted packed (x << 32) | z rows in a
// new pool buffer *out; returns the row count.
// known_total: the number of set bits when the caller knows it (no read-back), else UINT64_MAX
uint64_t bitmap_emit(Ctx *ctx, const uint64_t *bits, uint32_t nv, uint64_t words, uint64_t **out, int prof_kind,
                     uint64_t known_total = UINT64_MAX);

// Dense-domain fixpoint of a program whose rules are chains of binary
// relations: rule r derives head(v0, vk) from path[0](v0, v1), ...,
// path[k-1](v_{k-1}, v_k), atom j read forward or, when backward, with its
// columns swapped.  keys[p] / rows[p] are the canonical packed rows of every
// predicate (idb[p] marks rule heads; their rows are the initial contents),
// every id < domain.  Semi-naive iteration with the seed / delta-variant /
// iteration-count semantics of the join route; results are canonical packed
// rows per IDB predicate in out / out_n.
struct ChainAtom { int pred; bool backward; };
struct ChainRule { int head; std::vector<ChainAtom> path; };
void chain_fixpoint(Ctx *ctx, const std::vector<ChainRule> &rules, uint32_t n_preds, const std::vector<char> &idb,
                    const std::vector<const uint64_t *> &keys, const std::vector<uint64_t> &rows, uint32_t domain,
                    uint64_t max_iter, std::vector<uint64_t *> &out, std::vector<uint64_t> &out_n,
                    uint64_t *iterations, std::vector<uint64_t> &deltas);
// Bytes of device memory chain_fixpoint keeps for its bitmaps.
uint64_t chain_fixpoint_bytes(const std::vector<ChainRule> &rules, const std::vector<char> &idb, uint32_t domain);

// Arrow IPC stream codec for relations of 1..4 UInt32 columns (arrow_ipc.cpp,
// host code).  decode checks the stream and returns pointers to the column
// value buffers inside it (one schema, exactly one record batch); encode
// writes schema + one batch + end-of-stream.
struct IpcColumns {
    uint32_t arity = 0;
    uint64_t rows = 0;
    std::vector<const uint8_t *> cols;  // rows * 4 bytes each, possibly unaligned
    std::vector<std::string> names;
};
void ipc_decode_u32(const uint8_t *stream, uint64_t len, IpcColumns &out);
std::vector<uint8_t> ipc_encode_u32(const uint32_t *const *cols, uint32_t arity, uint64_t rows,
                                    const char *const *names);

// small helpers
inline unsigned grid_for(uint64_t n, unsigned block, unsigned cap) {
    uint64_t g = (n + block - 1) / block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (unsigned)g;
}
void fill_u32(Ctx *ctx, uint32_t *p, uint32_t v, uint64_t n);
// (cap: runs past it are counted in *d_count but not written)
void select_runs(Ctx *ctx, const uint64_t *k, uint64_t n, uint32_t *run_key, uint64_t *run_start,
                 uint64_t *d_count, const uint64_t *d_n = nullptr, const uint32_t *stop = nullptr,
                 uint64_t cap = ~0ull);
// Keys sorted by their high word: rows sharing it with a neighbour (key,
// position), then among those the group heads (key; gsel[position] = group
// number; hpos, when set, receives each head's position).
void select_group_members(Ctx *ctx, const uint64_t *k, uint64_t n, uint64_t *mkeys, uint64_t *mpos,
                          uint64_t *d_count);
void select_group_heads(Ctx *ctx, const uint64_t *mkeys, uint64_t nm, const uint64_t *mpos, uint64_t *hkeys,
                        int32_t *gsel, uint64_t *d_count, const uint64_t *d_n = nullptr, uint64_t *hpos = nullptr);
void sort_state_release(Ctx *ctx);
void select_state_release(Ctx *ctx);
// Exclusive scan of u64 counts in place, one pass; the exact total goes to
// *d_total (device).  The prefixes are exact while the total is below
// SCAN64_EXACT; a caller checks the total before using them.
constexpr uint64_t SCAN64_EXACT = 1ull << 39;
void scan_u64_inplace(Ctx *ctx, uint64_t *a, uint64_t n, uint64_t *d_total, const uint32_t *stop = nullptr);
// Zero-fills gathered into one launch (up to FILL_MAX_RANGES ranges each):
// add() records a range, flush() launches them in stream order.
constexpr int FILL_MAX_RANGES = 16;
struct FillBatch {
    Ctx *ctx;
    std::vector<std::pair<uint64_t *, uint64_t>> r;
    explicit FillBatch(Ctx *c) : ctx(c) {}
    void add(uint64_t *p, uint64_t n) {
        if (p && n) r.push_back({p, n});
    }
    void flush();
};
void fill_u64(Ctx *ctx, uint64_t *p, uint64_t v, uint64_t n);
void pack_columns(Ctx *ctx, const uint32_t *c0, const uint32_t *c1, uint64_t n, uint64_t *out);
void unpack_column(Ctx *ctx, const uint64_t *w, int hi, uint64_t n, uint32_t *out);
void swap_words(Ctx *ctx, const uint64_t *in, uint64_t n, uint64_t *out);  // (c0,c1) -> (c1,c0)
void low_words(Ctx *ctx, const uint64_t *in, uint64_t n, uint32_t *out);
int is_sorted_u64(Ctx *ctx, const uint64_t *k, uint64_t n, int strict);

}  // namespace xh
