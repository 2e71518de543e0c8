// Stream compaction, adjacent-compare dedup, sorted set difference and
// merge-path merge for gfx950.
//
// Replaces, on sorted packed u64 keys:
//   - mark_unique_full_row_bytewise + scan + compact_bytes_by_mask
//     (kernels/dedup.cu:306-345, scan.cu:133-270, filter.cu:902-942;
//     relational.rs:1558-1677) with ONE pass: flags, per-tile count,
//     decoupled look-back for the tile's output offset, ordered write;
//   - diff_via_deterministic_set's binary-search mark + scan + compact
//     (relational.rs:1311-1428, dedup.cu:515-565) with the same pass whose
//     flag is "unique and not in B", where each tile first narrows B to the
//     window spanned by its own first and last key;
//   - union_gpu's concat + full re-sort (relational.rs:822-999) with a
//     merge-path merge of the two sorted inputs.
#include "internal.hpp"
#include "short_runs.hpp"
#include <type_traits>

namespace xh {

namespace {

// Plain selections: 16 waves x 16 rows per lane, 16,384-row tiles (measured
// against 256/512-thread blocks and 8-64 rows per lane).  Selections that
// stage a window of a second array keep 8,192-row tiles, whose windows fit the
// LDS cap more often.
#ifndef XH_SEL_BLOCK
#define XH_SEL_BLOCK 1024
#endif
#ifndef XH_SEL_WIN_BLOCK
#define XH_SEL_WIN_BLOCK 512
#endif
#ifndef XH_SEL_ITEMS
#define XH_SEL_ITEMS 16
#endif
constexpr int SEL_BLOCK = XH_SEL_BLOCK;
constexpr int SEL_ITEMS = XH_SEL_ITEMS;
constexpr int SEL_WIN_BLOCK = XH_SEL_WIN_BLOCK;
// block, waves and tile rows of k_select<Sel>
template <class Sel>
struct SelShape {
    static constexpr int block = Sel::kWindow ? SEL_WIN_BLOCK : SEL_BLOCK;
    static constexpr int waves = block / WAVE;
    static constexpr uint64_t tile = (uint64_t)block * SEL_ITEMS;
};

// look-back status word: [63:40] epoch, [39] inclusive, [38:0] value
constexpr uint64_t LB_INC = 1ull << 39;
constexpr uint64_t LB_VAL = LB_INC - 1;

__device__ __forceinline__ uint64_t lb_load(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void lb_store(uint64_t *p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

// Exclusive prefix of the tile aggregates before `tile`, computed by one full
// wave that inspects 64 predecessors at a time.
__device__ uint64_t lookback_wave(const uint64_t *status, uint64_t tile, uint64_t epoch_tag, int lane) {
    uint64_t prefix = 0;
    int64_t j = (int64_t)tile - 1;
    while (j >= 0) {
        int64_t idx = j - lane;
        bool ready, inc;
        uint64_t val;
        if (idx >= 0) {
            uint64_t s = lb_load(status + idx);
            ready = (s & ~(LB_INC | LB_VAL)) == epoch_tag;
            inc = ready && (s & LB_INC);
            val = ready ? (s & LB_VAL) : 0;
        } else {
            ready = true; inc = true; val = 0;
        }
        uint64_t inc_mask = __ballot(inc);
        uint64_t nready = __ballot(!ready);
        if (inc_mask) {
            int f = __builtin_ctzll(inc_mask);
            uint64_t upto = (f == 63) ? ~0ull : ((2ull << f) - 1ull);
            if (nready & upto) continue;  // spin until the window up to the closest inclusive entry is ready
            prefix += wave_sum_u64(lane <= f ? val : 0ull);
            break;
        }
        if (nready) continue;
        prefix += wave_sum_u64(val);
        j -= WAVE;
    }
    return prefix;
}

// Dynamic LDS of window selections (SelDiff): the tile's window of B.
extern __shared__ uint64_t sel_window[];

// Generic single-pass selection.  Sel supplies:
//   static constexpr bool kWindow: false, or true for a selection that needs
//        a window of a second sorted array (then setup runs on all lanes of
//        wave 0, followed by a barrier)
//   __device__ void setup(uint64_t tile_first_idx, uint64_t tile_last_idx, uint64_t *smem, int lane)
//        (thread 0 only unless kWindow)
//   __device__ bool flag(uint64_t idx, uint64_t key, uint64_t prev_key, const uint64_t *smem)
//        (prev_key = in[idx - 1], meaningful for idx > 0)
//   kWindow selections instead: members<BLOCK, ITEMS>(keys, ...) (every
//        thread; bit r = key r is in the window) and
//        flag_member(idx, key, prev_key, member)
//   __device__ void emit(uint64_t pos, uint64_t idx, uint64_t key)
// A predicate that also reads the following row declares kNext = true and
// provides flag_next(idx, key, prev, next); next is 0 past the last row.
template <class S, class = void>
struct sel_next : std::false_type {};
template <class S>
struct sel_next<S, std::void_t<decltype(S::kNext)>> : std::bool_constant<S::kNext> {};

template <class Sel>
__global__ __launch_bounds__(SelShape<Sel>::block) void k_select(const uint64_t *__restrict__ in, uint64_t n, Sel sel,
                                                      uint64_t *__restrict__ d_count, uint64_t *status,
                                                      uint64_t epoch_tag, unsigned long long *ticket,
                                                      unsigned long long ticket_base, uint64_t ntiles,
                                                      const uint64_t *d_n, const uint32_t *stop) {
    __shared__ uint64_t s_tile;
    __shared__ uint64_t s_prefix;
    constexpr int SEL_WAVES = SelShape<Sel>::waves;
    constexpr uint64_t SEL_TILE = SelShape<Sel>::tile;
    __shared__ uint32_t s_wc[SEL_WAVES];
    __shared__ uint64_t s_sel[8];
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    // A row count on the device (d_n; n is then the bound the tiles' scratch
    // was sized for) makes the launch persistent: a grid of a few blocks per
    // CU takes tickets from a zeroed counter (ticket_base 0) until they pass
    // the tiles that hold rows, so its cost follows the real count, not the
    // bound; the last tile that holds rows (tile 0 when there are none)
    // writes the count.  Otherwise every block takes one ticket, from the
    // context's counter.  A stop raised by an earlier launch of a queued
    // iteration (it cannot change while this kernel runs) ends every block.
    const bool persist = d_n != nullptr;
    if (persist) {
        if (stop && *stop) return;
        n = *d_n < n ? *d_n : n;
        const uint64_t used = n ? (n + SEL_TILE - 1) / SEL_TILE : 1;
        ntiles = used < ntiles ? used : ntiles;
        if (blockIdx.x >= ntiles) return;  // more blocks than tiles: these take no ticket
    }
    for (;;) {
    if (tid == 0) s_tile = atomicAdd(ticket, 1ull) - ticket_base;
    __syncthreads();
    const uint64_t tile = s_tile;
    if (tile >= ntiles) {
        if (persist && tid == 0) persist_done(ticket, gridDim.x < ntiles ? gridDim.x : ntiles);
        return;
    }
    if constexpr (!Sel::kWindow) {
        if (tid == 0) {
            uint64_t first = tile * SEL_TILE, last = first + SEL_TILE;
            if (last > n) last = n;
            if (first < last) sel.setup(first, last - 1, s_sel, 0);
        }
        __syncthreads();
    } else {
        if (wave == 0) {
            uint64_t first = tile * SEL_TILE, last = first + SEL_TILE;
            if (last > n) last = n;
            if (first < last) {
                sel.setup(first, last - 1, s_sel, lane);
            } else if (lane == 0) {  // a tile past the rows: empty windows
                s_sel[0] = s_sel[1] = s_sel[3] = s_sel[4] = 0;
                s_sel[2] = s_sel[5] = 1;
            }
        }
        __syncthreads();
    }
    const uint64_t wbase = tile * SEL_TILE + (uint64_t)wave * (SEL_ITEMS * WAVE);
    const uint64_t lt_mask = (1ull << lane) - 1ull;
    uint64_t k[SEL_ITEMS];
    uint64_t fl = 0;  // bit r = flag of item r
    uint32_t wc = 0;
#pragma unroll
    for (int r = 0; r < SEL_ITEMS; ++r) {
        uint64_t idx = wbase + (uint64_t)r * WAVE + lane;
        k[r] = idx < n ? in[idx] : 0ull;
    }
    // predecessor of item r: lane-1 of the same round, lane 63 of the previous
    // round for lane 0, one extra load for the wave's first item
    uint64_t first_prev = (wbase > 0 && wbase <= n) ? in[wbase - 1] : 0ull;
    // successor likewise: lane+1 of the same round, lane 0 of the next round
    // for lane 63, one extra load after the wave's last item
    uint64_t last_next = 0;
    if constexpr (sel_next<Sel>::value) {
        const uint64_t e = wbase + (uint64_t)SEL_ITEMS * WAVE;
        last_next = e < n ? in[e] : 0ull;
    }
    uint32_t member = 0;  // window selections: bit r = key r is in the window
    if constexpr (Sel::kWindow) member = sel.template members<SelShape<Sel>::block, SEL_ITEMS>(k, wbase, n, s_sel, tid, lane);
#pragma unroll
    for (int r = 0; r < SEL_ITEMS; ++r) {
        uint64_t idx = wbase + (uint64_t)r * WAVE + lane;
        uint64_t up = __shfl_up(k[r], 1, WAVE);
        uint64_t carry = (r > 0) ? __shfl(k[r > 0 ? r - 1 : 0], WAVE - 1, WAVE) : first_prev;
        uint64_t prev = lane ? up : carry;
        bool f;
        if constexpr (sel_next<Sel>::value) {
            uint64_t down = __shfl_down(k[r], 1, WAVE);
            uint64_t ncarry = (r + 1 < SEL_ITEMS) ? __shfl(k[r + 1 < SEL_ITEMS ? r + 1 : r], 0, WAVE) : last_next;
            f = idx < n && sel.flag_next(idx, k[r], prev, lane < WAVE - 1 ? down : ncarry);
        } else if constexpr (Sel::kWindow) {
            f = idx < n && sel.flag_member(idx, k[r], prev, (member >> r) & 1u);
        } else {
            f = idx < n && sel.flag(idx, k[r], prev, s_sel);
        }
        if (f) fl |= 1ull << r;
        wc += (uint32_t)__popcll(__ballot(f));
    }
    if (lane == 0) s_wc[wave] = wc;
    __syncthreads();
    uint64_t tile_cnt = 0, wpre = 0;
#pragma unroll
    for (int w = 0; w < SEL_WAVES; ++w) {
        if (w < wave) wpre += s_wc[w];
        tile_cnt += s_wc[w];
    }
    if (wave == 0) {
        if (tid == 0) lb_store(status + tile, epoch_tag | (tile == 0 ? LB_INC : 0ull) | tile_cnt);
        uint64_t prefix = tile ? lookback_wave(status, tile, epoch_tag, lane) : 0ull;
        if (tid == 0) {
            if (tile) lb_store(status + tile, epoch_tag | LB_INC | (prefix + tile_cnt));
            s_prefix = prefix;
            if (tile == ntiles - 1) *d_count = prefix + tile_cnt;
        }
    }
    __syncthreads();
    uint64_t pos = s_prefix + wpre;
#pragma unroll
    for (int r = 0; r < SEL_ITEMS; ++r) {
        bool f = (fl >> r) & 1ull;
        uint64_t m = __ballot(f);
        if (f) sel.emit(pos + (uint64_t)__popcll(m & lt_mask), wbase + (uint64_t)r * WAVE + lane, k[r]);
        pos += (uint64_t)__popcll(m);
    }
    if (!persist) return;
    __syncthreads();  // the next tile reuses the shared words
    }
}

__device__ __forceinline__ uint64_t lower_bound_u64(const uint64_t *a, uint64_t lo, uint64_t hi, uint64_t key) {
    while (lo < hi) {
        uint64_t mid = lo + ((hi - lo) >> 1);
        if (a[mid] < key) lo = mid + 1; else hi = mid;
    }
    return lo;
}
__device__ __forceinline__ uint64_t upper_bound_u64(const uint64_t *a, uint64_t lo, uint64_t hi, uint64_t key) {
    while (lo < hi) {
        uint64_t mid = lo + ((hi - lo) >> 1);
        if (a[mid] <= key) lo = mid + 1; else hi = mid;
    }
    return lo;
}

struct SelUnique {
    const uint64_t *in;
    uint64_t *out;
    static constexpr bool kWindow = false;
    __device__ void setup(uint64_t, uint64_t, uint64_t *, int) const {}
    __device__ bool flag(uint64_t idx, uint64_t key, uint64_t prev, const uint64_t *) const {
        return idx == 0 || prev != key;
    }
    __device__ void emit(uint64_t pos, uint64_t, uint64_t key) const { out[pos] = key; }
};

// unique rows and, beside them, their low words (a join build's payloads)
struct SelUniqueLow {
    const uint64_t *in;
    uint64_t *out;
    uint32_t *low;
    static constexpr bool kWindow = false;
    __device__ void setup(uint64_t, uint64_t, uint64_t *, int) const {}
    __device__ bool flag(uint64_t idx, uint64_t key, uint64_t prev, const uint64_t *) const {
        return idx == 0 || prev != key;
    }
    __device__ void emit(uint64_t pos, uint64_t, uint64_t key) const {
        out[pos] = key;
        low[pos] = (uint32_t)key;
    }
};

// First position p in a[lo, hi) with !(a[p] < key) (UPPER: !(a[p] <= key)),
// by all 64 lanes of a wave: each round probes 64 evenly spaced positions and
// keeps the segment where the predicate turns, so a search over 2^30 keys
// takes 5 rounds of one load each instead of 30 dependent loads.
template <bool UPPER>
__device__ uint64_t wave_bound(const uint64_t *a, uint64_t lo, uint64_t hi, uint64_t key, int lane) {
    auto before = [&](uint64_t v) { return UPPER ? v <= key : v < key; };
    while (hi - lo > (uint64_t)WAVE) {
        const uint64_t step = (hi - lo + WAVE - 1) / WAVE;
        const uint64_t pr = lo + (uint64_t)lane * step;
        const uint64_t m = __ballot(pr < hi && before(a[pr]));  // lanes 0..c-1 (monotone)
        const int c = __popcll(m);
        if (c == 0) return lo;
        const uint64_t nlo = lo + (uint64_t)(c - 1) * step + 1;  // probe c-1 is before the bound
        const uint64_t nhi = lo + (uint64_t)c * step;             // probe c (if any) is not
        lo = nlo;
        hi = nhi < hi ? nhi : hi;
    }
    const uint64_t pr = lo + (uint64_t)lane;
    return lo + (uint64_t)__popcll(__ballot(pr < hi && before(a[pr])));
}

// unique (optional) and not a member of sorted b.  The tile's window of b
// (from its first key's lower bound to its last key's upper bound) comes from
// k_diff_windows, which finds every tile's window at once before the selection
// (a tile that searched its own would wait on 10 dependent rounds of loads
// before reading anything), or, for selections of fewer than DIFF_WINDOW_PASS
// tiles (where the extra launch costs more), is found by the tile's wave 0.
// A window of at most WIN_STREAM_PER_ROW keys per row of the tile (or
// of at most WIN_CAP keys) is streamed through LDS in chunks of WIN_CAP keys
// (one coalesced read of the window; each key is looked up in the chunk whose
// range holds it, in 13 fixed steps); a larger window is searched in HBM, one
// binary search per key, so that a small delta never streams a large b.
constexpr uint32_t WIN_CAP = 8192;             // keys per chunk (64 KB of dynamic LDS)
constexpr uint64_t WIN_STREAM_PER_ROW = 16;    // streamed window keys per row of the tile, at most
constexpr uint64_t DIFF_WINDOW_PASS = 256;     // tiles from which the windows come from k_diff_windows
// Membership of a tile's keys in the window [s0, s1) of sorted b: streamed
// through LDS in chunks of WIN_CAP keys, or searched in HBM.  Bit r: key k[r]
// (row wbase + r * WAVE + lane, below n) is in b.  Every thread of the block
// calls it (the streamed window has barriers).
//
// Each search is binary lifting from the largest power of two not above the
// window's length (pos = keys below k[r]); a lane runs SEARCH_GROUP of its
// keys' searches in lockstep, so that their loads are independent and in
// flight together instead of one chain of dependent loads per key (groups of 4
// keep the selection at 4 waves per SIMD: 119 VGPRs, none spilled).  The load
// index is clamped into the window, so every load is in bounds and none is
// predicated.  In LDS a group whose 4 x 64 keys all fall outside
// the chunk's range is skipped (a wave-uniform branch).
constexpr int SEARCH_GROUP = 4;
template <int BLOCK, int ITEMS>
__device__ uint32_t window_members(const uint64_t *b, uint64_t s0, uint64_t s1, bool streamed,
                                   const uint64_t (&k)[ITEMS], uint64_t wbase, uint64_t n, int tid, int lane) {
    static_assert(ITEMS % SEARCH_GROUP == 0, "search groups split the lane's items");
    uint32_t m = 0;
    if (streamed) {
        for (uint64_t c0 = s0; c0 < s1; c0 += WIN_CAP) {
            const uint32_t len = (uint32_t)(s1 - c0 < WIN_CAP ? s1 - c0 : WIN_CAP);
            __syncthreads();  // the previous chunk is no longer read
            batched_copy<BLOCK, 8>(
                len, tid, [&](uint32_t i) { return b[c0 + i]; }, [&](uint32_t i, uint64_t v) { sel_window[i] = v; });
            __syncthreads();
            const uint64_t lo_k = sel_window[0], hi_k = sel_window[len - 1];
            const uint32_t top = 1u << (31 - __builtin_clz(len));
#pragma unroll
            for (int g = 0; g < ITEMS; g += SEARCH_GROUP) {
                bool act[SEARCH_GROUP];
                bool any = false;
#pragma unroll
                for (int j = 0; j < SEARCH_GROUP; ++j) {
                    const uint64_t key = k[g + j];
                    act[j] = wbase + (uint64_t)(g + j) * WAVE + lane < n && key >= lo_k && key <= hi_k;
                    any |= act[j];
                }
                if (__ballot(any) == 0) continue;
                uint32_t pos[SEARCH_GROUP];
#pragma unroll
                for (int j = 0; j < SEARCH_GROUP; ++j) pos[j] = 0;
                for (uint32_t step = top; step > 0; step >>= 1) {
                    uint64_t v[SEARCH_GROUP];
#pragma unroll
                    for (int j = 0; j < SEARCH_GROUP; ++j) {
                        const uint32_t q = pos[j] + step;
                        v[j] = sel_window[(q <= len ? q : len) - 1];
                    }
#pragma unroll
                    for (int j = 0; j < SEARCH_GROUP; ++j)
                        if (pos[j] + step <= len && v[j] < k[g + j]) pos[j] += step;
                }
#pragma unroll
                for (int j = 0; j < SEARCH_GROUP; ++j) {
                    const uint64_t v = sel_window[pos[j] < len ? pos[j] : len - 1];
                    if (act[j] && pos[j] < len && v == k[g + j]) m |= 1u << (g + j);
                }
            }
        }
    } else if (s1 > s0) {
        const uint64_t len = s1 - s0;
        const uint64_t top = 1ull << (63 - __builtin_clzll(len));
#pragma unroll
        for (int g = 0; g < ITEMS; g += SEARCH_GROUP) {
            uint64_t pos[SEARCH_GROUP];
#pragma unroll
            for (int j = 0; j < SEARCH_GROUP; ++j) pos[j] = 0;
            for (uint64_t step = top; step > 0; step >>= 1) {
                uint64_t v[SEARCH_GROUP];
#pragma unroll
                for (int j = 0; j < SEARCH_GROUP; ++j) {
                    const uint64_t q = pos[j] + step;
                    v[j] = b[s0 + (q <= len ? q : len) - 1];
                }
#pragma unroll
                for (int j = 0; j < SEARCH_GROUP; ++j)
                    if (pos[j] + step <= len && v[j] < k[g + j]) pos[j] += step;
            }
#pragma unroll
            for (int j = 0; j < SEARCH_GROUP; ++j) {
                const bool valid = wbase + (uint64_t)(g + j) * WAVE + lane < n;
                if (valid && pos[j] < len && b[s0 + pos[j]] == k[g + j]) m |= 1u << (g + j);
            }
        }
    }
    return m;
}

// Unique (optional) and not a member of sorted b, nor of the optional second
// sorted array b2 (the two runs of a relation kept as a base run and a recent
// run).  b's windows come from k_diff_windows or the tile's own wave search
// (above); b2's from the tile's wave search.
template <bool UNIQ>
struct SelDiff {
    static constexpr bool kWindow = true;
    const uint64_t *in;
    const uint64_t *b;
    uint64_t nb;
    uint64_t *out;
    const uint64_t *win;  // [2t], [2t + 1]: window of tile t (nullptr: searched by the tile)
    uint64_t tile_rows;
    const uint64_t *d_nb;  // optional: b's row count on the device (nb is then its bound)
    const uint64_t *b2 = nullptr;  // optional second array, its bound and device count
    uint64_t nb2 = 0;
    const uint64_t *d_nb2 = nullptr;
    // s[0], s[1]: window [s0, s1) of b; s[2]: 1 when it is streamed through LDS; s[3..5] the same for b2
    __device__ void setup(uint64_t first, uint64_t last, uint64_t *s, int lane) const {
        uint64_t s0, s1;
        if (win) {
            const uint64_t t = first / tile_rows;
            s0 = win[2 * t];
            s1 = win[2 * t + 1];
        } else {
            const uint64_t m = d_nb && *d_nb < nb ? *d_nb : nb;
            s0 = wave_bound<false>(b, 0, m, in[first], lane);
            s1 = wave_bound<true>(b, s0, m, in[last], lane);
        }
        uint64_t t0 = 0, t1 = 0;
        if (b2) {
            const uint64_t m2 = d_nb2 && *d_nb2 < nb2 ? *d_nb2 : nb2;
            t0 = wave_bound<false>(b2, 0, m2, in[first], lane);
            t1 = wave_bound<true>(b2, t0, m2, in[last], lane);
        }
        if (lane == 0) {
            const uint64_t rows = last - first + 1;
            s[0] = s0;
            s[1] = s1;
            s[2] = (s1 - s0 <= WIN_CAP || s1 - s0 <= WIN_STREAM_PER_ROW * rows) ? 1u : 0u;
            s[3] = t0;
            s[4] = t1;
            s[5] = (t1 - t0 <= WIN_CAP || t1 - t0 <= WIN_STREAM_PER_ROW * rows) ? 1u : 0u;
        }
    }
    template <int BLOCK, int ITEMS>
    __device__ uint32_t members(const uint64_t (&k)[ITEMS], uint64_t wbase, uint64_t n, const uint64_t *s,
                                int tid, int lane) const {
        // one loop over the arrays, not two inlined copies: the selection keeps
        // 4 waves per SIMD (2 blocks per CU beside their LDS windows)
        uint32_t m = 0;
        const int arrays = b2 ? 2 : 1;
        for (int a = 0; a < arrays; ++a) {
            const uint64_t *arr = a ? b2 : b;
            const uint64_t *w = s + 3 * a;
            m |= window_members<BLOCK, ITEMS>(arr, w[0], w[1], w[2] != 0, k, wbase, n, tid, lane);
        }
        return m;
    }
    __device__ bool flag_member(uint64_t idx, uint64_t key, uint64_t prev, bool member) const {
        if (UNIQ && idx != 0 && prev == key) return false;
        return !member;
    }
    __device__ void emit(uint64_t pos, uint64_t, uint64_t key) const { out[pos] = key; }
};

// win[2t] = lower bound of tile t's first row in b, win[2t + 1] = upper bound
// of its last row: a thread per bound, all of them in flight at once (the top
// levels of the searches are shared and stay in cache)
__global__ __launch_bounds__(256) void k_diff_windows(const uint64_t *__restrict__ in, uint64_t n,
                                                      const uint64_t *__restrict__ b, uint64_t nb, uint64_t tile_rows,
                                                      uint64_t tiles, uint64_t *__restrict__ win,
                                                      const uint64_t *d_n, const uint64_t *d_nb,
                                                      const uint32_t *stop) {
    const uint64_t q = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= 2 * tiles) return;
    if (stop && *stop) return;
    // device row counts (queued iterations) replace the bounds the grid was sized for
    if (d_n && *d_n < n) n = *d_n;
    if (d_nb && *d_nb < nb) nb = *d_nb;
    const uint64_t t = q >> 1, first = t * tile_rows;
    if (first >= n) {  // a tile past the rows: an empty window
        win[q] = 0;
        return;
    }
    if (q & 1) {
        const uint64_t last = (first + tile_rows < n ? first + tile_rows : n) - 1;
        win[q] = upper_bound_u64(b, 0, nb, in[last]);
    } else {
        win[q] = lower_bound_u64(b, 0, nb, in[first]);
    }
}

// keys different from one value (the occupied slots of a hash table)
struct SelNotValue {
    uint64_t v;
    uint64_t *out;
    static constexpr bool kWindow = false;
    __device__ void setup(uint64_t, uint64_t, uint64_t *, int) const {}
    __device__ bool flag(uint64_t, uint64_t key, uint64_t, const uint64_t *) const { return key != v; }
    __device__ void emit(uint64_t pos, uint64_t, uint64_t key) const { out[pos] = key; }
};

// Grouped candidates over a small value domain (every low word below
// 64 * words), each group one run of equal high word x (select_runs): a block
// marks the group's low words in an LDS bitmap and x's row of R in a second
// one, and writes the values set in the first and not in the second,
// ascending, from the group's first position; the group's other positions
// get `hole`.  Every group is unique and sorted and has none of R's rows;
// compacted (select_not_value), the groups give the sorted delta.  x's row of
// R comes from R's runs (a base run of known size and a recent run counted on
// the device; found by four wave searches) or, with rin, from R as a bit
// matrix (`words` u64 words per row), and then R after the iteration, the row
// with the group's values added, goes to the same row of rout (each row
// belongs to one group; rows without a group are copied by the caller).
constexpr int GB_BLOCK = 512;
// x's rows of R (base and recent runs) into an LDS bitmap; every thread calls it
__device__ void rows_to_lds_bits(uint32_t x, const uint64_t *__restrict__ base, uint64_t nbase,
                                 const uint64_t *__restrict__ recent, uint64_t nrec, uint32_t limit,
                                 unsigned long long *rb, uint64_t *s_rng, int tid, int lane, int wave) {
    if (wave < 4) {  // x's rows: [x << 32, (x + 1) << 32) in the base run (waves 0, 1) and the recent run
        const uint64_t *a = wave < 2 ? base : recent;
        const uint64_t an = wave < 2 ? nbase : nrec;
        const uint64_t key = ((uint64_t)x + (uint64_t)(wave & 1)) << 32;
        const uint64_t pos = an ? wave_bound<false>(a, 0, an, key, lane) : 0ull;
        if (lane == 0) s_rng[wave] = pos;
    }
    __syncthreads();
    for (uint64_t i = s_rng[0] + (uint64_t)tid; i < s_rng[1]; i += GB_BLOCK) {
        const uint32_t z = (uint32_t)base[i];
        if (z < limit) atomicOr(&rb[z >> 6], 1ull << (z & 63u));
    }
    for (uint64_t i = s_rng[2] + (uint64_t)tid; i < s_rng[3]; i += GB_BLOCK) {
        const uint32_t z = (uint32_t)recent[i];
        if (z < limit) atomicOr(&rb[z >> 6], 1ull << (z & 63u));
    }
}
// R as a bit matrix (rows 0 .. domain - 1, `words` u64 words each), from its runs
__global__ __launch_bounds__(GB_BLOCK) void k_rows_to_bits(const uint64_t *__restrict__ base, uint64_t nbase,
                                                           const uint64_t *__restrict__ recent, uint64_t nrec,
                                                           uint32_t domain, uint32_t words, uint64_t *__restrict__ bits) {
    extern __shared__ unsigned long long gb_bits[];
    __shared__ uint64_t s_rng[4];
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    for (uint32_t x = blockIdx.x; x < domain; x += gridDim.x) {
        for (uint32_t w = (uint32_t)tid; w < words; w += GB_BLOCK) gb_bits[w] = 0ull;
        rows_to_lds_bits(x, base, nbase, recent, nrec, 64u * words, gb_bits, s_rng, tid, lane, wave);
        __syncthreads();
        for (uint32_t w = (uint32_t)tid; w < words; w += GB_BLOCK) bits[(uint64_t)x * words + w] = gb_bits[w];
        __syncthreads();
    }
}
__global__ __launch_bounds__(GB_BLOCK) void k_group_bitmap_diff(
    const uint64_t *__restrict__ cand, const uint64_t *d_cand, uint64_t cand_bound,
    const uint32_t *__restrict__ run_key, const uint64_t *__restrict__ run_start, const uint64_t *d_nruns,
    uint64_t runs_bound, const uint64_t *__restrict__ base, uint64_t nbase, const uint64_t *__restrict__ recent,
    const uint64_t *d_nrecent, uint64_t recent_bound, uint32_t words, uint64_t hole, uint64_t *__restrict__ slots,
    const uint64_t *__restrict__ rin, uint64_t *__restrict__ rout, const uint32_t *stop) {
    extern __shared__ unsigned long long gb_bits[];  // [0, words): the group's values, [words, 2 words): R's
    __shared__ uint64_t s_rng[4];
    __shared__ uint32_t s_wsum[GB_BLOCK / WAVE];
    if (stop && *stop) return;
    const uint64_t n = *d_cand < cand_bound ? *d_cand : cand_bound;
    const uint64_t nruns = *d_nruns < runs_bound ? *d_nruns : runs_bound;
    const uint64_t nrec = *d_nrecent < recent_bound ? *d_nrecent : recent_bound;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    const uint32_t limit = 64u * words;
    unsigned long long *cb = gb_bits, *rb = gb_bits + words;
    for (uint64_t g = blockIdx.x; g < nruns; g += gridDim.x) {
        const uint32_t x = run_key[g];
        const uint64_t st = run_start[g], en = g + 1 < nruns ? run_start[g + 1] : n;
        for (uint32_t w = (uint32_t)tid; w < words; w += GB_BLOCK) {
            cb[w] = 0ull;
            rb[w] = rin ? rin[(uint64_t)x * words + w] : 0ull;
        }
        if (!rin) rows_to_lds_bits(x, base, nbase, recent, nrec, limit, rb, s_rng, tid, lane, wave);
        __syncthreads();
        for (uint64_t i = st + (uint64_t)tid; i < en; i += GB_BLOCK) {
            const uint32_t z = (uint32_t)cand[i];
            if (z < limit) atomicOr(&cb[z >> 6], 1ull << (z & 63u));
        }
        __syncthreads();
        if (rout)  // R after this iteration: the row with the group's values added
            for (uint32_t w = (uint32_t)tid; w < words; w += GB_BLOCK) rout[(uint64_t)x * words + w] = rb[w] | cb[w];
        // thread t takes words [t * per, (t + 1) * per): its new values' count, a block scan, then the values
        const uint32_t per = (words + GB_BLOCK - 1) / GB_BLOCK;
        uint32_t cnt = 0;
        for (uint32_t k = 0; k < per; ++k) {
            const uint32_t w = (uint32_t)tid * per + k;
            if (w < words) cnt += (uint32_t)__popcll(cb[w] & ~rb[w]);
        }
        uint32_t incl = cnt;
#pragma unroll
        for (int o = 1; o < WAVE; o <<= 1) {
            const uint32_t t = __shfl_up(incl, o, WAVE);
            if (lane >= o) incl += t;
        }
        if (lane == WAVE - 1) s_wsum[wave] = incl;
        __syncthreads();
        uint32_t pre = incl - cnt, total = 0;
#pragma unroll
        for (int q = 0; q < GB_BLOCK / WAVE; ++q) {
            if (q < wave) pre += s_wsum[q];
            total += s_wsum[q];
        }
        uint64_t pos = st + pre;
        const uint64_t hi = (uint64_t)x << 32;
        for (uint32_t k = 0; k < per; ++k) {
            const uint32_t w = (uint32_t)tid * per + k;
            if (w >= words) break;
            unsigned long long bits = cb[w] & ~rb[w];
            while (bits) {
                slots[pos++] = hi | (uint64_t)(w * 64u + (uint32_t)__builtin_ctzll(bits));
                bits &= bits - 1ull;
            }
        }
        for (uint64_t i = st + total + (uint64_t)tid; i < en; i += GB_BLOCK) slots[i] = hole;
        __syncthreads();  // the bitmaps and s_rng are reused by the next group
    }
}

struct SelFlags {
    const uint8_t *flags;
    uint64_t *out;
    static constexpr bool kWindow = false;
    __device__ void setup(uint64_t, uint64_t, uint64_t *, int) const {}
    __device__ bool flag(uint64_t idx, uint64_t, uint64_t, const uint64_t *) const { return flags[idx] != 0; }
    __device__ void emit(uint64_t pos, uint64_t, uint64_t key) const { out[pos] = key; }
};

// run starts of the high word (join build)
// Rows of keys sorted by their high word that share it with a neighbour
// (groups of >= 2 rows): key and position.
struct SelGroupMembers {
    const uint64_t *in;
    uint64_t n;
    uint64_t *out_key, *out_pos;
    static constexpr bool kWindow = false;
    static constexpr bool kNext = true;
    __device__ void setup(uint64_t, uint64_t, uint64_t *, int) const {}
    __device__ bool flag_next(uint64_t idx, uint64_t key, uint64_t prev, uint64_t next) const {
        const uint32_t h = (uint32_t)(key >> 32);
        return (idx > 0 && (uint32_t)(prev >> 32) == h) || (idx + 1 < n && (uint32_t)(next >> 32) == h);
    }
    __device__ void emit(uint64_t pos, uint64_t idx, uint64_t key) const {
        out_key[pos] = key;
        out_pos[pos] = idx;
    }
};
// Group heads among the member rows above: the head key and, at the head's
// original row, its group number in the row-group selector.
struct SelGroupHeads {
    const uint64_t *mpos;
    uint64_t *out_key;
    int32_t *gsel;
    uint64_t *out_pos;  // optional: the head's original row
    static constexpr bool kWindow = false;
    __device__ void setup(uint64_t, uint64_t, uint64_t *, int) const {}
    __device__ bool flag(uint64_t idx, uint64_t key, uint64_t prev, const uint64_t *) const {
        return idx == 0 || (uint32_t)(prev >> 32) != (uint32_t)(key >> 32);
    }
    __device__ void emit(uint64_t pos, uint64_t idx, uint64_t key) const {
        out_key[pos] = key;
        const uint64_t p = mpos[idx];
        gsel[p] = (int32_t)pos;
        if (out_pos) out_pos[pos] = p;
    }
};

struct SelRuns {
    const uint64_t *in;
    uint32_t *run_key;
    uint64_t *run_start;
    uint64_t cap = ~0ull;  // runs past it are counted, not written
    static constexpr bool kWindow = false;
    __device__ void setup(uint64_t, uint64_t, uint64_t *, int) const {}
    __device__ bool flag(uint64_t idx, uint64_t key, uint64_t prev, const uint64_t *) const {
        return idx == 0 || (prev >> 32) != (key >> 32);
    }
    __device__ void emit(uint64_t pos, uint64_t idx, uint64_t key) const {
        if (pos >= cap) return;
        run_key[pos] = (uint32_t)(key >> 32);
        run_start[pos] = idx;
    }
};

// ---- exclusive scan of u32, in place ----------------------------------------
// One pass with decoupled look-back (replaces the reference's three-phase
// recursive multiblock scan, scan.cu:133-270, provider/mod.rs:2192-2290).  A
// thread owns SCAN_ITEMS consecutive values (16-byte loads when the array is
// 16-byte aligned), scans them serially, the block scans the thread sums, and
// the tile's prefix comes from the look-back over earlier tiles.  Prefixes are
// u32 and wrap modulo 2^32 like the reference's u32 arithmetic; the exact u64
// total is accumulated separately (one atomic per tile).
constexpr int SCAN_BLOCK = 1024;
constexpr int SCAN_ITEMS = 16;
constexpr uint64_t SCAN_TILE = (uint64_t)SCAN_BLOCK * SCAN_ITEMS;

template <bool VEC>
__global__ __launch_bounds__(SCAN_BLOCK) void k_scan_u32(uint32_t *a, uint64_t n, uint64_t *status,
                                                         uint64_t epoch_tag, unsigned long long *ticket,
                                                         unsigned long long ticket_base,
                                                         unsigned long long *d_total) {
    __shared__ uint64_t s_tile;
    __shared__ uint32_t s_prefix;
    __shared__ uint32_t s_wsum[SCAN_BLOCK / WAVE];
    __shared__ unsigned long long s_wsum64[SCAN_BLOCK / WAVE];
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    if (tid == 0) s_tile = atomicAdd(ticket, 1ull) - ticket_base;
    __syncthreads();
    const uint64_t tile = s_tile;
    const uint64_t base = tile * SCAN_TILE + (uint64_t)tid * SCAN_ITEMS;
    uint32_t v[SCAN_ITEMS];
    if (VEC && base + SCAN_ITEMS <= n) {
        const uint4 *q = reinterpret_cast<const uint4 *>(a + base);
#pragma unroll
        for (int k = 0; k < SCAN_ITEMS / 4; ++k) {
            const uint4 x = q[k];
            v[4 * k] = x.x; v[4 * k + 1] = x.y; v[4 * k + 2] = x.z; v[4 * k + 3] = x.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < SCAN_ITEMS; ++k) v[k] = base + k < n ? a[base + k] : 0u;
    }
    uint32_t sum = 0;
    unsigned long long sum64 = 0;
#pragma unroll
    for (int k = 0; k < SCAN_ITEMS; ++k) {
        const uint32_t x = v[k];
        v[k] = sum;  // thread-local exclusive prefix
        sum += x;
        sum64 += x;
    }
    // wave scan of the thread sums
    uint32_t incl = sum;
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
        const uint32_t t = __shfl_up(incl, o, WAVE);
        if (lane >= o) incl += t;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum64 += __shfl_xor(sum64, o, WAVE);
    if (lane == WAVE - 1) s_wsum[wave] = incl;
    if (lane == 0) s_wsum64[wave] = sum64;
    __syncthreads();
    uint32_t wpre = 0, tile_sum = 0;
    unsigned long long tile_sum64 = 0;
#pragma unroll
    for (int w = 0; w < SCAN_BLOCK / WAVE; ++w) {
        if (w < wave) wpre += s_wsum[w];
        tile_sum += s_wsum[w];
        tile_sum64 += s_wsum64[w];
    }
    if (wave == 0) {
        if (tid == 0) {
            lb_store(status + tile, epoch_tag | (tile == 0 ? LB_INC : 0ull) | tile_sum);
            atomicAdd(d_total, tile_sum64);
        }
        // the look-back sums prefixes in u64; only their value modulo 2^32 is used
        const uint64_t prefix = tile ? lookback_wave(status, tile, epoch_tag, lane) : 0ull;
        if (tid == 0) {
            if (tile) lb_store(status + tile, epoch_tag | LB_INC | (uint32_t)(prefix + tile_sum));
            s_prefix = (uint32_t)prefix;
        }
    }
    __syncthreads();
    const uint32_t off = s_prefix + wpre + (incl - sum);
    if (VEC && base + SCAN_ITEMS <= n) {
        uint4 *q = reinterpret_cast<uint4 *>(a + base);
#pragma unroll
        for (int k = 0; k < SCAN_ITEMS / 4; ++k)
            q[k] = make_uint4(off + v[4 * k], off + v[4 * k + 1], off + v[4 * k + 2], off + v[4 * k + 3]);
    } else {
#pragma unroll
        for (int k = 0; k < SCAN_ITEMS; ++k)
            if (base + k < n) a[base + k] = off + v[k];
    }
}

// ---- exclusive scan of u64 counts, in place --------------------------------
// The probe's per-tile output counts.  Same single pass as k_scan_u32; the
// look-back words carry 39-bit values, and the exact u64 total is added up
// separately (one atomic per tile): a caller whose total reaches 2^39 must not
// use the prefixes (no bag that large fits a device anyway).
constexpr int SCAN64_BLOCK = 1024;
constexpr int SCAN64_ITEMS = 8;
constexpr uint64_t SCAN64_TILE = (uint64_t)SCAN64_BLOCK * SCAN64_ITEMS;

__global__ __launch_bounds__(SCAN64_BLOCK) void k_scan_u64(uint64_t *a, uint64_t n, uint64_t *status,
                                                           uint64_t epoch_tag, unsigned long long *ticket,
                                                           unsigned long long ticket_base,
                                                           unsigned long long *d_total, const uint32_t *stop) {
    __shared__ uint64_t s_tile;
    __shared__ uint64_t s_prefix;
    __shared__ uint64_t s_wsum[SCAN64_BLOCK / WAVE];
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    if (tid == 0) s_tile = atomicAdd(ticket, 1ull) - ticket_base;
    if (stop && *stop) return;  // after the ticket (see k_select)
    __syncthreads();
    const uint64_t tile = s_tile;
    const uint64_t base = tile * SCAN64_TILE + (uint64_t)tid * SCAN64_ITEMS;
    uint64_t v[SCAN64_ITEMS];
#pragma unroll
    for (int k = 0; k < SCAN64_ITEMS; ++k) v[k] = base + k < n ? a[base + k] : 0ull;
    uint64_t sum = 0;
#pragma unroll
    for (int k = 0; k < SCAN64_ITEMS; ++k) {
        const uint64_t x = v[k];
        v[k] = sum;
        sum += x;
    }
    uint64_t incl = sum;
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
        const uint64_t t = __shfl_up(incl, o, WAVE);
        if (lane >= o) incl += t;
    }
    if (lane == WAVE - 1) s_wsum[wave] = incl;
    __syncthreads();
    uint64_t wpre = 0, tile_sum = 0;
#pragma unroll
    for (int w = 0; w < SCAN64_BLOCK / WAVE; ++w) {
        if (w < wave) wpre += s_wsum[w];
        tile_sum += s_wsum[w];
    }
    if (wave == 0) {
        if (tid == 0) {
            lb_store(status + tile, epoch_tag | (tile == 0 ? LB_INC : 0ull) | (tile_sum & LB_VAL));
            if (tile_sum) atomicAdd(d_total, (unsigned long long)tile_sum);
        }
        const uint64_t prefix = tile ? lookback_wave(status, tile, epoch_tag, lane) : 0ull;
        if (tid == 0) {
            if (tile) lb_store(status + tile, epoch_tag | LB_INC | ((prefix + tile_sum) & LB_VAL));
            s_prefix = prefix;
        }
    }
    __syncthreads();
    const uint64_t off = s_prefix + wpre + (incl - sum);
#pragma unroll
    for (int k = 0; k < SCAN64_ITEMS; ++k)
        if (base + k < n) a[base + k] = off + v[k];
}

// ---- merge path -----------------------------------------------------------
constexpr int MRG_BLOCK = 256;
constexpr int MRG_ITEMS = 8;
constexpr int MRG_TILE = MRG_BLOCK * MRG_ITEMS;

// number of a-elements among the first d outputs of the stable merge (a first on ties)
__device__ __forceinline__ uint64_t merge_path(const uint64_t *a, uint64_t na, const uint64_t *b, uint64_t nb,
                                               uint64_t d) {
    uint64_t lo = d > nb ? d - nb : 0, hi = d < na ? d : na;
    while (lo < hi) {
        uint64_t mid = lo + ((hi - lo) >> 1);
        if (a[mid] <= b[d - 1 - mid]) lo = mid + 1; else hi = mid;
    }
    return lo;
}

// split[t] = merge_path at diagonal min(t * MRG_TILE, na + nb), one thread per
// tile boundary: the binary searches of all tiles run side by side instead of
// two dependent ~log2(n)-load chains at the start of every merge block
// Queued iterations give the row counts on the device (d_na, d_nb replace the
// bounds na, nb the grid was sized for), a stop flag, and a skip word: a merge
// whose *skip is zero writes nothing (an iteration that derived nothing keeps
// its relation where it is).
struct MergeDev {
    const uint64_t *d_na = nullptr, *d_nb = nullptr, *skip = nullptr;
    const uint32_t *stop = nullptr;
    __device__ bool off() const { return (stop && *stop) || (skip && *skip == 0); }
    __device__ void counts(uint64_t &na, uint64_t &nb) const {
        if (d_na && *d_na < na) na = *d_na;
        if (d_nb && *d_nb < nb) nb = *d_nb;
    }
};

__global__ void k_merge_partition(const uint64_t *__restrict__ a, uint64_t na, const uint64_t *__restrict__ b,
                                  uint64_t nb, uint64_t tiles, uint64_t *__restrict__ split, MergeDev dv) {
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t > tiles || dv.off()) return;
    dv.counts(na, nb);
    const uint64_t total = na + nb, d = t * MRG_TILE < total ? t * MRG_TILE : total;
    split[t] = merge_path(a, na, b, nb, d);
}

__global__ __launch_bounds__(MRG_BLOCK) void k_merge(const uint64_t *__restrict__ a, uint64_t na,
                                                     const uint64_t *__restrict__ b, uint64_t nb,
                                                     const uint64_t *__restrict__ split, uint64_t *__restrict__ out,
                                                     MergeDev dv) {
    __shared__ uint64_t s[MRG_TILE];
    __shared__ uint64_t s_split[2];
    const int tid = threadIdx.x;
    if (dv.off()) return;
    dv.counts(na, nb);
    const uint64_t total = na + nb;
    // with device counts a grid of a few blocks per CU strides over the real tiles
    const bool persist = dv.d_na || dv.d_nb;
    for (uint64_t tile = blockIdx.x;; tile += gridDim.x) {
    const uint64_t d0 = tile * MRG_TILE;
    if (d0 >= total) return;
    const uint64_t d1 = (d0 + MRG_TILE < total) ? d0 + MRG_TILE : total;
    if (tid < 2) s_split[tid] = split[tile + tid];
    __syncthreads();
    // For sorted inputs the splits are monotone and the clamp changes nothing; for inputs that are not
    // sorted it keeps the tile's ranges inside a and b (and LDS) instead of inverting them.
    const uint64_t a0 = s_split[0];
    uint64_t a1 = s_split[1];
    {
        const uint64_t lo1 = d1 > nb && d1 - nb > a0 ? d1 - nb : a0;
        const uint64_t hi1 = a0 + (d1 - d0) < na ? a0 + (d1 - d0) : na;
        a1 = a1 < lo1 ? lo1 : (a1 > hi1 ? hi1 : a1);
    }
    const uint32_t la = (uint32_t)(a1 - a0), len = (uint32_t)(d1 - d0), lb = len - la;
    const uint64_t b0 = d0 - a0;
    batched_copy<MRG_BLOCK, MRG_ITEMS>(
        len, tid, [&](uint32_t i) { return i < la ? a[a0 + i] : b[b0 + (i - la)]; },
        [&](uint32_t i, uint64_t v) { s[i] = v; });
    __syncthreads();
    const uint64_t *sa = s, *sb = s + la;
    uint32_t td = tid * MRG_ITEMS;
    uint64_t r[MRG_ITEMS];
    uint32_t cnt = 0;
    if (td < len) {
        uint32_t ia = (uint32_t)merge_path(sa, la, sb, lb, td);
        uint32_t ib = td - ia;
#pragma unroll
        for (int j = 0; j < MRG_ITEMS; ++j) {
            if (td + j < len) {
                bool take_a = ib >= lb || (ia < la && sa[ia] <= sb[ib]);
                r[j] = take_a ? sa[ia] : sb[ib];
                ia += take_a; ib += !take_a;
                ++cnt;
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < MRG_ITEMS; ++j)
        if ((uint32_t)j < cnt) s[td + j] = r[j];
    __syncthreads();
    for (uint32_t i = tid; i < len; i += MRG_BLOCK) out[d0 + i] = s[i];
    if (!persist) return;
    __syncthreads();  // s is reused by the next tile
    }
}

// profiling of launches sized by bounds: the real row counts (up to two
// device counts, each clamped to its bound), weighted, added to a work counter
__global__ void k_work_rows(unsigned long long *work, const uint64_t *d_a, uint64_t a, uint32_t wa, const uint64_t *d_b,
                            uint64_t b, uint32_t wb, const uint64_t *skip, const uint32_t *stop) {
    if ((stop && *stop) || (skip && *skip == 0)) return;
    if (d_a && *d_a < a) a = *d_a;
    if (d_b && *d_b < b) b = *d_b;
    atomicAdd(work, (unsigned long long)(a * wa + b * wb));
}

// ---- helpers --------------------------------------------------------------
__global__ void k_pack(const uint32_t *__restrict__ c0, const uint32_t *__restrict__ c1, uint64_t n,
                       uint64_t *__restrict__ out) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = ((uint64_t)c0[i] << 32) | (c1 ? c1[i] : 0u);
}
__global__ void k_unpack(const uint64_t *__restrict__ w, int hi, uint64_t n, uint32_t *__restrict__ out) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = hi ? (uint32_t)(w[i] >> 32) : (uint32_t)w[i];
}
__global__ void k_swap(const uint64_t *__restrict__ in, uint64_t n, uint64_t *__restrict__ out) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        uint64_t k = in[i];
        out[i] = (k << 32) | (k >> 32);
    }
}
__global__ void k_unsorted(const uint64_t *__restrict__ k, uint64_t n, int strict, uint32_t *flag) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i + 1 < n; i += stride) {
        bool bad = strict ? !(k[i] < k[i + 1]) : (k[i] > k[i + 1]);
        if (bad) *flag = 1u;
    }
}

// Sort of short runs fused with the adjacent-compare unique, for the
// high-word route of a full-key sort + dedup.  Each tile places the runs it owns (short_runs_place), keeps a placed key when it
// differs from the key placed before it (the first place of the tile starts
// a run, whose high word differs from every earlier key), counts the kept
// keys, takes its output offset from decoupled look-back over the tiles'
// counts and writes them there, coalesced.  Reads every key once (plus the
// 1 + SRU_MAX halo per tile) and writes only the unique keys.  `work`
// (profiling, optional) counts the written keys.  Tile = workgroup index, so
// a tile waits only on tiles of lower index, which started before it when
// workgroups start in index order (the radix pass's condition (1)); with
// `ticket` the tile is the block's start ticket and the look-back holds
// without that condition.  On C3 (2^28 keys, 65,536 tiles) the ticket's one
// device-wide atomic per tile cost 0.09-0.25 ms of 1.67 (two A/B runs).
constexpr int SRU_BLOCK = 512, SRU_CORE = 4096, SRU_MAX = 256;  // 256 x 2048 measured 10 % slower
using SruTile = ShortRunTile<SRU_BLOCK, SRU_CORE, SRU_MAX>;
__global__ __launch_bounds__(SRU_BLOCK) void k_short_runs_unique(const uint64_t *__restrict__ in, uint64_t n,
                                                                 uint64_t *__restrict__ out, uint64_t *d_count,
                                                                 uint64_t *long_run, uint64_t *status,
                                                                 uint64_t epoch_tag, unsigned long long *ticket,
                                                                 unsigned long long ticket_base, uint64_t ntiles,
                                                                 unsigned long long *work) {
    __shared__ SruTile t;
    __shared__ uint64_t s_tile, s_prefix;
    __shared__ uint32_t s_wc[SRU_BLOCK / WAVE];
    constexpr int IT = SruTile::ITEMS;  // a wave covers WAVE * IT consecutive places
    static_assert(SRU_BLOCK * IT >= SRU_CORE + SRU_MAX, "the waves must cover the placed range");
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    if (ticket) {
        if (tid == 0) s_tile = atomicAdd(ticket, 1ull) - ticket_base;
        __syncthreads();
    }
    const uint64_t tile = ticket ? s_tile : (uint64_t)blockIdx.x;
    short_runs_place<SRU_BLOCK, SRU_CORE, SRU_MAX>(in, n, tile * SRU_CORE, t, long_run);
    const uint32_t pmin = t.pmin, pmax = t.pmax;
    const uint32_t wb = pmin + (uint32_t)wave * (WAVE * IT);
    uint32_t fl = 0, wc = 0;
#pragma unroll
    for (int r = 0; r < IT; ++r) {
        const uint32_t i = wb + (uint32_t)(r * WAVE + lane);
        const bool f = pmin != 0xFFFFFFFFu && i < pmax && (i == pmin || t.hi[i] != t.hi[i - 1] || t.lo[i] != t.lo[i - 1]);
        if (f) fl |= 1u << r;
        wc += (uint32_t)__popcll(__ballot(f));
    }
    if (lane == 0) s_wc[wave] = wc;
    __syncthreads();
    uint64_t tile_cnt = 0, wpre = 0;
#pragma unroll
    for (int w = 0; w < SRU_BLOCK / WAVE; ++w) {
        if (w < wave) wpre += s_wc[w];
        tile_cnt += s_wc[w];
    }
    if (wave == 0) {
        if (tid == 0) lb_store(status + tile, epoch_tag | (tile == 0 ? LB_INC : 0ull) | tile_cnt);
        const uint64_t prefix = tile ? lookback_wave(status, tile, epoch_tag, lane) : 0ull;
        if (tid == 0) {
            if (tile) lb_store(status + tile, epoch_tag | LB_INC | (prefix + tile_cnt));
            s_prefix = prefix;
            if (tile == ntiles - 1) *d_count = prefix + tile_cnt;
            if (work && tile_cnt) atomicAdd(&work[blockIdx.x & (Ctx::PROF_WORK_SPREAD - 1)], tile_cnt);
        }
    }
    __syncthreads();
    const uint64_t lt_mask = (1ull << lane) - 1ull;
    uint64_t pos = s_prefix + wpre;
#pragma unroll
    for (int r = 0; r < IT; ++r) {
        const bool f = (fl >> r) & 1u;
        const uint64_t m = __ballot(f);
        if (f) {
            const uint32_t i = wb + (uint32_t)(r * WAVE + lane);
            out[pos + (uint64_t)__popcll(m & lt_mask)] = ((uint64_t)t.hi[i] << 32) | t.lo[i];
        }
        pos += (uint64_t)__popcll(m);
    }
}

// Segment sort of a large keys-only sort whose keys two digit passes have
// ordered by their top 16 bits: a segment is the keys of 2^gshift consecutive
// top-16-bit values (gshift chosen by the caller for about 4,096 keys per
// segment of uniform input), and every segment is sorted by the rest of the key
// on chip, one 1024-thread block per segment (two per CU).  This is the hybrid
// radix sort of Stehle and Jacobsen ("A Memory Bandwidth-Efficient Hybrid
// Radix Sort on GPUs", SIGMOD 2017): global digit passes until every bucket
// fits on chip, then one on-chip sort per bucket.  The sort is of whole keys
// only, so equal keys need no stable order, and one counting pass places the
// segment: each key takes a slot of its bin of the 12 bits below the segment's
// (bits 36 + gshift .. 47 + gshift, 4,096 bins, about one key each for uniform
// keys) by an LDS atomic, the bins' starts come from a block scan, and every
// key is then ranked inside its bin by the whole key (a bin is the run of keys
// that agree from bit 36 + gshift up).  The segment is written at its place
// (sort), or its unique keys at an offset from decoupled look-back over the
// segments' counts (sort + unique).  A segment of more than SEG_MAX keys, or a
// bin of more than SEG_RUN_MAX keys that are not all equal, raises *long_run:
// the block then counts zero and writes nothing, and the caller sorts the keys
// by every digit instead.
constexpr int SEG_BLOCK = 1024, SEG_ITEMS = 5, SEG_MAX = SEG_BLOCK * SEG_ITEMS, SEG_RUN_MAX = 256, SEG_RANK_BATCH = 4;
constexpr int SEG_WAVES = SEG_BLOCK / WAVE;
constexpr int SEG_BIN_BITS = 12, SEG_BINS = 1 << SEG_BIN_BITS;
constexpr uint32_t SEG_COUNT = 1u << 16;  // top-16-bit values
static_assert((uint64_t)SEG_MAX == SORT_SEGMENT_MAX, "segment capacity");
static_assert(SEG_BINS % SEG_BLOCK == 0, "bins per thread");

// A segment is the keys of 2^gshift consecutive top-16-bit values (their bits
// 48 + gshift and up agree): bounds[s] = index of the first key of segment s
// or a later one (keys ordered by their top 16 bits), bounds[nseg] = n.
__global__ void k_seg_bounds(const uint64_t *__restrict__ keys, uint64_t n, uint32_t nseg, int gshift,
                             uint64_t *__restrict__ bounds) {
    const uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s > nseg) return;
    uint64_t lo = 0, hi = n;
    if (s == nseg) {
        lo = n;
    } else {
        const uint64_t target = (uint64_t)s << (48 + gshift);
        while (lo < hi) {
            const uint64_t mid = (lo + hi) >> 1;
            if (keys[mid] < target) lo = mid + 1;
            else hi = mid;
        }
    }
    bounds[s] = lo;
}

struct SegSmem {
    uint64_t key[SEG_MAX];              // the segment's keys at their place
    uint32_t bin[SEG_BINS];             // key counts, then the bins' starts
    uint8_t uf[SEG_MAX];                // 1 at the place of the first of every group of equal keys
    uint32_t wsum[SEG_WAVES];
    uint32_t wc[SEG_WAVES];
    uint64_t prefix;
    uint32_t tile;
    uint32_t bad;
};

// One block per segment: block index, or (UNIQUE with `ticket`) the block's
// start ticket, so that a segment's look-back waits only on segments whose
// blocks started before it.  UNIQUE: the unique keys go to out at their
// offset and their total to *d_count; otherwise the segment's keys go to out
// at the segment's place.
template <bool UNIQUE>
__global__ __launch_bounds__(SEG_BLOCK) __attribute__((amdgpu_waves_per_eu(8))) void k_seg_sort(const uint64_t *__restrict__ in,
                                                        const uint64_t *__restrict__ bounds, uint64_t *__restrict__ out,
                                                        uint64_t *d_count, uint64_t *long_run, uint64_t *status,
                                                        uint64_t epoch_tag, unsigned long long *ticket,
                                                        unsigned long long ticket_base, uint32_t nseg, int gshift,
                                                        unsigned long long *work) {
    __shared__ SegSmem sm;
    // the bins take the 12 bits below the segment's own (bits 36 + gshift .. 47 + gshift)
    const int bin_shift = 48 - SEG_BIN_BITS + gshift;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    constexpr int BPT = SEG_BINS / SEG_BLOCK;  // consecutive bins per thread in the scan
#pragma unroll
    for (int q = 0; q < BPT; ++q) sm.bin[tid * BPT + q] = 0u;
    if (tid == 0) {
        sm.bad = 0;
        if (UNIQUE && ticket) sm.tile = (uint32_t)(atomicAdd(ticket, 1ull) - ticket_base);
    }
    __syncthreads();
    const uint32_t seg = (UNIQUE && ticket) ? __builtin_amdgcn_readfirstlane(sm.tile) : blockIdx.x;
    const uint64_t a = bounds[seg], b = bounds[seg + 1];
    const bool too_big = b - a > (uint64_t)SEG_MAX;
    const uint32_t len = too_big ? 0u : (uint32_t)(b - a);
    if (too_big && tid == 0) *long_run = 1ull;

    // the segment's keys in registers (key r of a thread: tid + r * SEG_BLOCK),
    // each with its slot in its bin
    uint64_t k[SEG_ITEMS];
    uint32_t slot[SEG_ITEMS];
#pragma unroll
    for (int r = 0; r < SEG_ITEMS; ++r) {
        const uint32_t p = (uint32_t)(tid + r * SEG_BLOCK);
        k[r] = p < len ? in[a + p] : 0ull;
    }
#pragma unroll
    for (int r = 0; r < SEG_ITEMS; ++r) {
        const uint32_t p = (uint32_t)(tid + r * SEG_BLOCK);
        slot[r] = p < len ? atomicAdd(&sm.bin[(uint32_t)(k[r] >> bin_shift) & (SEG_BINS - 1)], 1u) : 0u;
    }
    __syncthreads();
    // exclusive scan of the bin counts: BPT consecutive bins per thread, then waves
    uint32_t c[BPT], run = 0;
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
        c[q] = sm.bin[tid * BPT + q];
        run += c[q];
    }
    uint32_t incl = run;
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
        const uint32_t t = __shfl_up(incl, o, WAVE);
        if (lane >= o) incl += t;
    }
    if (lane == WAVE - 1) sm.wsum[wave] = incl;
    __syncthreads();
    uint32_t start = incl - run;
#pragma unroll
    for (int w = 0; w < SEG_WAVES; ++w)
        if (w < wave) start += sm.wsum[w];
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
        sm.bin[tid * BPT + q] = start;
        start += c[q];
    }
    __syncthreads();
    // scatter to the bins: slot r of bin b goes to place start(b) + r
    uint32_t place[SEG_ITEMS];
#pragma unroll
    for (int r = 0; r < SEG_ITEMS; ++r) {
        const uint32_t p = (uint32_t)(tid + r * SEG_BLOCK);
        place[r] = 0u;
        if (p < len) {
            place[r] = sm.bin[(uint32_t)(k[r] >> bin_shift) & (SEG_BINS - 1)] + slot[r];
            sm.key[place[r]] = k[r];
        }
    }
    __syncthreads();
    // rank inside the bin (the run of keys that share bits 36..63) by (key,
    // place): the key's place in the segment; `moved` marks keys whose place
    // changes and `uniq` the first of every group of equal keys.  Every key's
    // bin bounds are read first, and a bin's first SEG_RANK_BATCH keys are
    // loaded together (most bins hold fewer).
    bool longr = false;
    uint32_t moved = 0, uniq = 0;
    uint32_t bst[SEG_ITEMS], bln[SEG_ITEMS];
#pragma unroll
    for (int r = 0; r < SEG_ITEMS; ++r) {
        const uint32_t p = (uint32_t)(tid + r * SEG_BLOCK);
        const uint32_t bn = (uint32_t)(k[r] >> bin_shift) & (SEG_BINS - 1);
        bst[r] = p < len ? sm.bin[bn] : 0u;
        bln[r] = p < len ? (bn + 1 < (uint32_t)SEG_BINS ? sm.bin[bn + 1] : len) - bst[r] : 0u;
    }
#pragma unroll
    for (int r = 0; r < SEG_ITEMS; ++r) {
        const uint32_t st = bst[r], ln = bln[r];
        if (ln < 2) {
            if (ln == 1) uniq |= 1u << r;
            continue;
        }
        if (ln > (uint32_t)SEG_RUN_MAX) {
            // a long bin is left as it is when all its keys are equal (any
            // order is sorted); the key at its start stands for them
            if (sm.key[st] != k[r]) longr = true;
            else if (place[r] == st) uniq |= 1u << r;
            continue;
        }
        uint32_t rk = 0;
        bool eq_before = false;
        uint64_t kj[SEG_RANK_BATCH];
#pragma unroll
        for (int u = 0; u < SEG_RANK_BATCH; ++u) {
            const uint32_t j = st + ((uint32_t)u < ln ? (uint32_t)u : ln - 1);
            kj[u] = sm.key[j];
        }
#pragma unroll
        for (int u = 0; u < SEG_RANK_BATCH; ++u) {
            const bool in = (uint32_t)u < ln, before = st + u < place[r];
            rk += (in && (kj[u] < k[r] || (kj[u] == k[r] && before))) ? 1u : 0u;
            eq_before |= in && kj[u] == k[r] && before;
        }
        for (uint32_t j = st + SEG_RANK_BATCH; j < st + ln; ++j) {
            const uint64_t x = sm.key[j];
            rk += (x < k[r] || (x == k[r] && j < place[r])) ? 1u : 0u;
            eq_before |= x == k[r] && j < place[r];
        }
        if (!eq_before) uniq |= 1u << r;
        if (st + rk != place[r]) {
            place[r] = st + rk;
            moved |= 1u << r;
        }
    }
    uint32_t wu = 0;
    if (UNIQUE) {
#pragma unroll
        for (int r = 0; r < SEG_ITEMS; ++r) wu += (uint32_t)__popcll(__ballot((uniq >> r) & 1u));
    }
    if (lane == 0) sm.wc[wave] = wu;
    if (__ballot(longr) != 0 && lane == 0) {
        sm.bad = 1u;
        *long_run = 1ull;
    }
    __syncthreads();  // every rank has read the bins; sm.bad and the counts are final
    const bool bad = sm.bad != 0u;
    uint64_t tile_cnt = 0;
    if (UNIQUE) {
#pragma unroll
        for (int w = 0; w < SEG_WAVES; ++w) tile_cnt += sm.wc[w];
        if (bad) tile_cnt = 0;
        // the segment's count is known: published before its keys are placed
        if (tid == 0) lb_store(status + seg, epoch_tag | (seg == 0 ? LB_INC : 0ull) | tile_cnt);
    }
    if (!bad) {
#pragma unroll
        for (int r = 0; r < SEG_ITEMS; ++r) {
            const uint32_t p = (uint32_t)(tid + r * SEG_BLOCK);
            if (UNIQUE && p < len) sm.uf[place[r]] = (uint8_t)((uniq >> r) & 1u);
            if (!((moved >> r) & 1u)) continue;
            sm.key[place[r]] = k[r];
        }
    }
    __syncthreads();
    const uint32_t wbase = (uint32_t)wave * (SEG_ITEMS * WAVE);
    const uint32_t n_out = bad ? 0u : len;
    if (!UNIQUE) {
        for (uint32_t i = tid; i < n_out; i += SEG_BLOCK) out[a + i] = sm.key[i];
        return;
    }
    // the unique keys in place order, counted per wave over consecutive places
    uint32_t fl = 0, wc = 0;
#pragma unroll
    for (int r = 0; r < SEG_ITEMS; ++r) {
        const uint32_t i = wbase + (uint32_t)(r * WAVE + lane);
        const bool f = i < n_out && sm.uf[i] != 0;
        if (f) fl |= 1u << r;
        wc += (uint32_t)__popcll(__ballot(f));
    }
    if (lane == 0) sm.wc[wave] = wc;
    __syncthreads();
    uint64_t wpre = 0;
#pragma unroll
    for (int w = 0; w < SEG_WAVES; ++w)
        if (w < wave) wpre += sm.wc[w];
    if (wave == 0) {
        const uint64_t prefix = seg ? lookback_wave(status, seg, epoch_tag, lane) : 0ull;
        if (tid == 0) {
            if (seg) lb_store(status + seg, epoch_tag | LB_INC | (prefix + tile_cnt));
            sm.prefix = prefix;
            if (seg == nseg - 1) *d_count = prefix + tile_cnt;
            if (work && tile_cnt) atomicAdd(&work[blockIdx.x & (Ctx::PROF_WORK_SPREAD - 1)], tile_cnt);
        }
    }
    __syncthreads();
    const uint64_t lt_mask = (1ull << lane) - 1ull;
    uint64_t pos = sm.prefix + wpre;
#pragma unroll
    for (int r = 0; r < SEG_ITEMS; ++r) {
        const bool f = (fl >> r) & 1u;
        const uint64_t m = __ballot(f);
        if (f) {
            const uint32_t i = wbase + (uint32_t)(r * WAVE + lane);
            out[pos + (uint64_t)__popcll(m & lt_mask)] = sm.key[i];
        }
        pos += (uint64_t)__popcll(m);
    }
}

}  // namespace

// ---- host wrappers ----------------------------------------------------------

struct SelectState {
    uint64_t *status = nullptr;
    uint64_t cap = 0;
    uint64_t epoch = 0;
};
static std::map<Ctx *, SelectState> g_sel_state;
static std::mutex g_sel_mu;

void select_state_release(Ctx *ctx) {
    std::lock_guard<std::mutex> g(g_sel_mu);
    auto it = g_sel_state.find(ctx);
    if (it == g_sel_state.end()) return;
    if (it->second.status) ctx->free(it->second.status);
    g_sel_state.erase(it);
}

// status buffer with >= tiles entries and a fresh epoch tag
static uint64_t *select_status(Ctx *ctx, uint64_t tiles, uint64_t *epoch_tag) {
    std::lock_guard<std::mutex> g(g_sel_mu);
    SelectState &st = g_sel_state[ctx];
    if (tiles > st.cap || st.epoch + 1 >= (1ull << 24)) {
        uint64_t cap = tiles > st.cap ? (tiles < 4096 ? 4096 : tiles + tiles / 4) : st.cap;
        if (st.status) ctx->free(st.status);
        st.status = static_cast<uint64_t *>(ctx->alloc(cap * sizeof(uint64_t)));
        fill_u64(ctx, st.status, 0ull, cap);
        st.cap = cap;
        st.epoch = 0;
    }
    st.epoch += 1;
    *epoch_tag = st.epoch << 40;
    return st.status;
}

// d_n (optional): the row count on the device, at most n, which is then only
// the bound the grid is sized for.  stop (optional): the stop flag of a queued
// iteration; a raised flag makes the launch do nothing (*d_count unwritten).
template <class Sel>
static void run_select(Ctx *ctx, const uint64_t *in, uint64_t n, const Sel &sel, uint64_t *d_count,
                       const uint64_t *d_n = nullptr, const uint32_t *stop = nullptr) {
    if (n == 0) {
        fill_u64(ctx, d_count, 0ull, 1);
        return;
    }
    constexpr uint64_t tile_rows = SelShape<Sel>::tile;
    uint64_t tiles = (n + tile_rows - 1) / tile_rows;
    XH_REQUIRE(tiles < (1ull << 31), XLOG_HIP_CAPACITY_OVERFLOW, "select: input too large");
    uint64_t tag;
    uint64_t *status = select_status(ctx, tiles, &tag);
    // tickets: one per block from the context's counter, or, for a persistent launch (device row
    // count), from a counter zeroed for it
    unsigned long long *tk = ctx->tickets + 1, tb = 0;
    unsigned grid = (unsigned)tiles;
    if (d_n) {
        tk = ctx->tickets + PERSIST_TICKET_SLOT;  // at zero: the last launch's last block reset it
        grid = persistent_grid(ctx, tiles, 8);
    } else {
        tb = ctx->take_tickets(1, tiles);
    }
    // 8 B per input row; with a device row count, counted on the device
    Prof prof(ctx, XLOG_HIP_KERNEL_SELECT, d_n ? 0.0 : 8.0 * (double)n);
    if (d_n) add_work_rows(ctx, prof.work(8.0), d_n, n, 1, nullptr, 0, 0, nullptr, stop);
    const size_t dyn = Sel::kWindow ? (size_t)WIN_CAP * sizeof(uint64_t) : 0;
    hipLaunchKernelGGL(k_select<Sel>, dim3(grid), dim3(SelShape<Sel>::block), dyn, ctx->stream, in, n, sel, d_count,
                       status, tag, tk, tb, tiles, d_n, stop);
    XH_CHECK_HIP(hipGetLastError());
}

void sort_short_runs_unique(Ctx *ctx, const uint64_t *in, uint64_t n, uint64_t *out, uint64_t *d_count,
                            uint64_t *d_long) {
    fill_u64(ctx, d_long, 0ull, 1);
    if (n == 0) {
        fill_u64(ctx, d_count, 0ull, 1);
        return;
    }
    const uint64_t tiles = (n + SRU_CORE - 1) / SRU_CORE;
    XH_REQUIRE(tiles < (1ull << 31), XLOG_HIP_CAPACITY_OVERFLOW, "short-run unique: input too large");
    uint64_t tag;
    uint64_t *status = select_status(ctx, tiles, &tag);
    unsigned long long *tk = sort_tickets() ? ctx->tickets + 1 : nullptr;
    const unsigned long long tb = tk ? ctx->take_tickets(1, tiles) : 0ull;
    // algorithmic bytes: every key read once, every unique key written once (counted on the device)
    Prof prof(ctx, XLOG_HIP_KERNEL_SORT_RUNS, 8.0 * (double)n);
    unsigned long long *work = prof.work(8.0);
    hipLaunchKernelGGL(k_short_runs_unique, dim3((unsigned)tiles), dim3(SRU_BLOCK), 0, ctx->stream, in, n, out, d_count,
                       d_long, status, tag, tk, tb, tiles, work);
    XH_CHECK_HIP(hipGetLastError());
}

void sort_top_segments(Ctx *ctx, const uint64_t *in, uint64_t n, uint64_t *out, uint64_t *d_count, uint64_t *d_long,
                       int gshift) {
    XH_REQUIRE(gshift >= 0 && gshift <= 8, XLOG_HIP_INVALID_ARG, "segment sort: group shift outside [0, 8]");
    fill_u64(ctx, d_long, 0ull, 1);
    if (n == 0) {
        if (d_count) fill_u64(ctx, d_count, 0ull, 1);
        return;
    }
    const uint32_t nseg = SEG_COUNT >> gshift;
    Buf<uint64_t> bounds(ctx, nseg + 1);
    hipLaunchKernelGGL(k_seg_bounds, dim3((nseg + 1 + 255) / 256), dim3(256), 0, ctx->stream, in, n, nseg, gshift,
                       bounds.p);
    XH_CHECK_HIP(hipGetLastError());
    if (d_count) {
        uint64_t tag;
        uint64_t *status = select_status(ctx, nseg, &tag);
        unsigned long long *tk = sort_tickets() ? ctx->tickets + 1 : nullptr;
        const unsigned long long tb = tk ? ctx->take_tickets(1, nseg) : 0ull;
        // algorithmic bytes: every key read once, every unique key written once (counted on the device)
        Prof prof(ctx, XLOG_HIP_KERNEL_SORT_SEGMENTS, 8.0 * (double)n);
        unsigned long long *work = prof.work(8.0);
        hipLaunchKernelGGL(k_seg_sort<true>, dim3(nseg), dim3(SEG_BLOCK), 0, ctx->stream, in, bounds.p, out,
                           d_count, d_long, status, tag, tk, tb, nseg, gshift, work);
    } else {
        Prof prof(ctx, XLOG_HIP_KERNEL_SORT_SEGMENTS, 16.0 * (double)n);  // every key read and written once
        hipLaunchKernelGGL(k_seg_sort<false>, dim3(nseg), dim3(SEG_BLOCK), 0, ctx->stream, in, bounds.p, out,
                           nullptr, d_long, nullptr, 0ull, nullptr, 0ull, nseg, gshift, nullptr);
    }
    XH_CHECK_HIP(hipGetLastError());
}

void select_unique(Ctx *ctx, const uint64_t *k, uint64_t n, uint64_t *out, uint64_t *d_count, const uint64_t *d_n) {
    run_select(ctx, k, n, SelUnique{k, out}, d_count, d_n);
}
void select_unique_low(Ctx *ctx, const uint64_t *k, uint64_t n, uint64_t *out, uint32_t *low, uint64_t *d_count) {
    run_select(ctx, k, n, SelUniqueLow{k, out, low}, d_count);
}
void select_unique_diff(Ctx *ctx, const uint64_t *k, uint64_t n, const uint64_t *b, uint64_t nb, uint64_t *out,
                        uint64_t *d_count) {
    if (nb == 0 || n == 0) { select_unique(ctx, k, n, out, d_count); return; }
    select_unique_diff_dev(ctx, k, n, nullptr, b, nb, nullptr, out, d_count, nullptr);
}
void add_work_rows(Ctx *ctx, unsigned long long *work, const uint64_t *d_a, uint64_t a, uint32_t wa, const uint64_t *d_b,
                   uint64_t b, uint32_t wb, const uint64_t *skip, const uint32_t *stop) {
    if (!work) return;
    hipLaunchKernelGGL(k_work_rows, dim3(1), dim3(1), 0, ctx->stream, work, d_a, a, wa, d_b, b, wb, skip, stop);
    XH_CHECK_HIP(hipGetLastError());
}

void select_unique_diff_dev(Ctx *ctx, const uint64_t *k, uint64_t n, const uint64_t *d_n, const uint64_t *b,
                            uint64_t nb, const uint64_t *d_nb, uint64_t *out, uint64_t *d_count, const uint32_t *stop) {
    select_unique_diff2_dev(ctx, k, n, d_n, b, nb, d_nb, nullptr, 0, nullptr, out, d_count, stop);
}
void select_unique_diff2_dev(Ctx *ctx, const uint64_t *k, uint64_t n, const uint64_t *d_n, const uint64_t *b,
                             uint64_t nb, const uint64_t *d_nb, const uint64_t *b2, uint64_t nb2, const uint64_t *d_nb2,
                             uint64_t *out, uint64_t *d_count, const uint32_t *stop) {
    if (n == 0) {
        fill_u64(ctx, d_count, 0ull, 1);
        return;
    }
    // b may be empty only when its count is on the device (an empty b of
    // known size takes select_unique): a window search then finds nothing
    constexpr uint64_t rows = SelShape<SelDiff<true>>::tile;
    const uint64_t tiles = (n + rows - 1) / rows;
    XH_REQUIRE(tiles < (1ull << 31), XLOG_HIP_CAPACITY_OVERFLOW, "select: input too large");
    Buf<uint64_t> win;
    if (tiles >= DIFF_WINDOW_PASS) {
        win = Buf<uint64_t>(ctx, 2 * tiles);
        hipLaunchKernelGGL(k_diff_windows, dim3((unsigned)((2 * tiles + 255) / 256)), dim3(256), 0, ctx->stream, k, n, b,
                           nb, rows, tiles, win.p, d_n, d_nb, stop);
        XH_CHECK_HIP(hipGetLastError());
    }
    SelDiff<true> sel{k, b, nb, out, win.p, rows, d_nb};
    sel.b2 = b2;
    sel.nb2 = nb2;
    sel.d_nb2 = d_nb2;
    run_select(ctx, k, n, sel, d_count, d_n, stop);
}
void select_not_value(Ctx *ctx, const uint64_t *k, uint64_t n, uint64_t v, uint64_t *out, uint64_t *d_count,
                      const uint64_t *d_n, const uint32_t *stop) {
    run_select(ctx, k, n, SelNotValue{v, out}, d_count, d_n, stop);
}
void rows_to_bits(Ctx *ctx, const uint64_t *base, uint64_t nbase, const uint64_t *recent, uint64_t nrec,
                  uint32_t domain, uint64_t *bits) {
    const uint32_t words = (domain + 63u) / 64u;
    XH_REQUIRE(words >= 1 && words <= 2048, XLOG_HIP_INVALID_ARG, "bit matrix: domain above 2^17");
    hipLaunchKernelGGL(k_rows_to_bits, dim3(persistent_grid(ctx, domain, 4)), dim3(GB_BLOCK), words * sizeof(uint64_t),
                       ctx->stream, base, nbase, recent, nrec, domain, words, bits);
    XH_CHECK_HIP(hipGetLastError());
}
void group_bitmap_diff_dev(Ctx *ctx, const uint64_t *cand, uint64_t cand_bound, const uint64_t *d_cand,
                           const uint32_t *run_key, const uint64_t *run_start, uint64_t runs_bound,
                           const uint64_t *d_nruns, const uint64_t *base, uint64_t nbase, const uint64_t *recent,
                           uint64_t recent_bound, const uint64_t *d_nrecent, uint32_t domain, uint64_t hole,
                           uint64_t *slots, const uint64_t *rin, uint64_t *rout, const uint32_t *stop) {
    if (cand_bound == 0 || runs_bound == 0) return;
    const uint32_t words = (domain + 63u) / 64u;
    XH_REQUIRE(words >= 1 && words <= 2048, XLOG_HIP_INVALID_ARG, "group bitmap difference: domain above 2^17");
    // the groups' and R's bytes, counted on the device (8 B per candidate read and per slot written)
    Prof prof(ctx, XLOG_HIP_KERNEL_SELECT, 0.0);
    add_work_rows(ctx, prof.work(16.0), d_cand, cand_bound, 1, nullptr, 0, 0, nullptr, stop);
    hipLaunchKernelGGL(k_group_bitmap_diff, dim3(persistent_grid(ctx, runs_bound, 4)), dim3(GB_BLOCK),
                       2 * words * sizeof(uint64_t), ctx->stream, cand, d_cand, cand_bound, run_key, run_start,
                       d_nruns, runs_bound, base, nbase, recent, d_nrecent, recent_bound, words, hole, slots, rin, rout,
                       stop);
    XH_CHECK_HIP(hipGetLastError());
}
// Rows run_key[0 .. *d_n) (at most bound) of one bit matrix copied to another
// (`words` u64 words per row): a block per row.
__global__ __launch_bounds__(256) void k_copy_group_rows(const uint32_t *__restrict__ run_key, const uint64_t *d_n,
                                                         uint64_t bound, uint32_t words,
                                                         const uint64_t *__restrict__ src, uint64_t *__restrict__ dst,
                                                         const uint32_t *stop) {
    if (stop && *stop) return;
    const uint64_t n = *d_n < bound ? *d_n : bound;
    for (uint64_t g = blockIdx.x; g < n; g += gridDim.x) {
        const uint64_t row = (uint64_t)run_key[g] * words;
        for (uint32_t w = threadIdx.x; w < words; w += blockDim.x) dst[row + w] = src[row + w];
    }
}
void copy_group_rows(Ctx *ctx, const uint32_t *run_key, const uint64_t *d_n, uint64_t bound, uint32_t domain,
                     const uint64_t *src, uint64_t *dst, const uint32_t *stop) {
    if (bound == 0) return;
    const uint32_t words = (domain + 63u) / 64u;
    Prof prof(ctx, XLOG_HIP_KERNEL_MERGE, 0.0);
    hipLaunchKernelGGL(k_copy_group_rows, dim3(persistent_grid(ctx, bound, 8)), dim3(256), 0, ctx->stream, run_key,
                       d_n, bound, words, src, dst, stop);
    XH_CHECK_HIP(hipGetLastError());
}
__global__ void k_rows_bits(const uint64_t *__restrict__ rows, const uint64_t *d_n, uint64_t bound, uint32_t words,
                            unsigned long long *__restrict__ bits, int clear, const uint32_t *stop) {
    if (stop && *stop) return;
    const uint64_t n = *d_n < bound ? *d_n : bound;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t w = rows[i];
        const uint64_t idx = (w >> 32) * words + ((uint32_t)w >> 6);
        if (clear) bits[idx] = 0ull;
        else atomicOr(&bits[idx], 1ull << ((uint32_t)w & 63u));
    }
}
void rows_bits(Ctx *ctx, const uint64_t *rows, const uint64_t *d_n, uint64_t bound, uint32_t words, uint64_t *bits,
               bool clear, const uint32_t *stop) {
    if (bound == 0) return;
    Prof prof(ctx, XLOG_HIP_KERNEL_SELECT, 0.0);
    hipLaunchKernelGGL(k_rows_bits, dim3(grid_for(bound, 256, 2048)), dim3(256), 0, ctx->stream, rows, d_n, bound,
                       words, reinterpret_cast<unsigned long long *>(bits), clear ? 1 : 0, stop);
    XH_CHECK_HIP(hipGetLastError());
}
void select_flags(Ctx *ctx, const uint64_t *k, const uint8_t *flags, uint64_t n, uint64_t *out, uint64_t *d_count) {
    run_select(ctx, k, n, SelFlags{flags, out}, d_count);
}
void select_group_members(Ctx *ctx, const uint64_t *k, uint64_t n, uint64_t *mkeys, uint64_t *mpos,
                          uint64_t *d_count) {
    run_select(ctx, k, n, SelGroupMembers{k, n, mkeys, mpos}, d_count);
}
void select_group_heads(Ctx *ctx, const uint64_t *mkeys, uint64_t nm, const uint64_t *mpos, uint64_t *hkeys,
                        int32_t *gsel, uint64_t *d_count, const uint64_t *d_n, uint64_t *hpos) {
    XH_REQUIRE(nm < (1ull << 31), XLOG_HIP_CAPACITY_OVERFLOW, "join: too many grouped probe rows");
    run_select(ctx, mkeys, nm, SelGroupHeads{mpos, hkeys, gsel, hpos}, d_count, d_n);
}
void select_runs(Ctx *ctx, const uint64_t *k, uint64_t n, uint32_t *run_key, uint64_t *run_start, uint64_t *d_count,
                 const uint64_t *d_n, const uint32_t *stop, uint64_t cap) {
    SelRuns sel{k, run_key, run_start};
    sel.cap = cap;
    run_select(ctx, k, n, sel, d_count, d_n, stop);
}

void scan_u64_inplace(Ctx *ctx, uint64_t *a, uint64_t n, uint64_t *d_total, const uint32_t *stop) {
    fill_u64(ctx, d_total, 0ull, 1);
    if (n == 0) return;
    const uint64_t tiles = (n + SCAN64_TILE - 1) / SCAN64_TILE;
    XH_REQUIRE(tiles < (1ull << 31), XLOG_HIP_CAPACITY_OVERFLOW, "scan: input too large");
    uint64_t tag;
    uint64_t *status = select_status(ctx, tiles, &tag);
    unsigned long long tb = ctx->take_tickets(1, tiles);
    hipLaunchKernelGGL(k_scan_u64, dim3((unsigned)tiles), dim3(SCAN64_BLOCK), 0, ctx->stream, a, n, status, tag,
                       ctx->tickets + 1, tb, reinterpret_cast<unsigned long long *>(d_total), stop);
    XH_CHECK_HIP(hipGetLastError());
}

void scan_u32_inplace(Ctx *ctx, uint32_t *a, uint64_t n, unsigned long long *d_total) {
    fill_u64(ctx, reinterpret_cast<uint64_t *>(d_total), 0ull, 1);
    if (n == 0) return;
    const uint64_t tiles = (n + SCAN_TILE - 1) / SCAN_TILE;
    XH_REQUIRE(tiles < (1ull << 31), XLOG_HIP_CAPACITY_OVERFLOW, "scan: input too large");
    uint64_t tag;
    uint64_t *status = select_status(ctx, tiles, &tag);
    unsigned long long tb = ctx->take_tickets(1, tiles);
    Prof prof(ctx, XLOG_HIP_KERNEL_SELECT, 8.0 * (double)n);  // reads and writes 4 B per value
    if ((reinterpret_cast<uintptr_t>(a) & 15u) == 0)
        hipLaunchKernelGGL(k_scan_u32<true>, dim3((unsigned)tiles), dim3(SCAN_BLOCK), 0, ctx->stream, a, n, status,
                           tag, ctx->tickets + 1, tb, d_total);
    else
        hipLaunchKernelGGL(k_scan_u32<false>, dim3((unsigned)tiles), dim3(SCAN_BLOCK), 0, ctx->stream, a, n, status,
                           tag, ctx->tickets + 1, tb, d_total);
    XH_CHECK_HIP(hipGetLastError());
}

// ---- the scan without allocation ---------------------------------------------
// Device scratch of the allocation-free scan: [0] tile ticket, [1] exact total,
// [2 ..] one look-back status word per tile.  It is a file-scope device array,
// so every GPU the library runs on holds its own copy from module load to
// process exit; its device address differs per GPU and is looked up once per
// device (scan_noalloc_init) with that device current.  The name `scratch` in
// host code is a host-side stand-in, never a device address: host code uses the
// looked-up pointer only.
constexpr uint64_t SCAN_NOALLOC_TILES = SCAN_NOALLOC_MAX / SCAN_TILE + 1;
static_assert(SCAN_NOALLOC_MAX % SCAN_TILE == 0, "whole tiles");
static __device__ __align__(256) uint64_t scratch[2 + SCAN_NOALLOC_TILES];

static std::mutex g_noalloc_mu;
static uint64_t *g_noalloc_ptr[64] = {nullptr};

void scan_noalloc_init(int device) {
    XH_REQUIRE(device >= 0 && device < 64, XLOG_HIP_INVALID_ARG, "device index above 63");
    std::lock_guard<std::mutex> g(g_noalloc_mu);
    if (g_noalloc_ptr[device]) return;
    void *p = nullptr;
    XH_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    XH_REQUIRE(p, XLOG_HIP_DEVICE_ERROR, "scratch symbol has no device address");
    g_noalloc_ptr[device] = static_cast<uint64_t *>(p);
}

void scan_u32_inplace_noalloc(Ctx *ctx, uint32_t *a, uint64_t n, uint64_t *total) {
    XH_REQUIRE(n <= SCAN_NOALLOC_MAX, XLOG_HIP_CAPACITY_OVERFLOW,
               "scan without allocation: n = " + std::to_string(n) + " exceeds the maximum " +
                   std::to_string(SCAN_NOALLOC_MAX));
    uint64_t *sp = nullptr;
    {
        std::lock_guard<std::mutex> g(g_noalloc_mu);
        sp = (ctx->device >= 0 && ctx->device < 64) ? g_noalloc_ptr[ctx->device] : nullptr;
    }
    XH_REQUIRE(sp, XLOG_HIP_DEVICE_ERROR, "scan without allocation: scratch not set up for this device");
    const uint64_t tiles = (n + SCAN_TILE - 1) / SCAN_TILE;
    // the ticket, the total and the status words of this call's tiles start at
    // zero (a kernel fill, no memset); status words carry a fixed epoch tag,
    // so a zeroed word reads as "not yet published"
    fill_u64(ctx, sp, 0ull, 2 + tiles);
    if (n) {
        unsigned long long *ticket = reinterpret_cast<unsigned long long *>(sp);
        unsigned long long *d_total = reinterpret_cast<unsigned long long *>(sp + 1);
        const uint64_t tag = 1ull << 40;
        if ((reinterpret_cast<uintptr_t>(a) & 15u) == 0)
            hipLaunchKernelGGL(k_scan_u32<true>, dim3((unsigned)tiles), dim3(SCAN_BLOCK), 0, ctx->stream, a, n,
                               sp + 2, tag, ticket, 0ull, d_total);
        else
            hipLaunchKernelGGL(k_scan_u32<false>, dim3((unsigned)tiles), dim3(SCAN_BLOCK), 0, ctx->stream, a, n,
                               sp + 2, tag, ticket, 0ull, d_total);
        XH_CHECK_HIP(hipGetLastError());
    }
    // the total comes back through the context's pinned staging (no allocation)
    XH_CHECK_HIP(hipMemcpyAsync(ctx->host_scalars, sp + 1, sizeof(uint64_t), hipMemcpyDeviceToHost, ctx->stream));
    ctx->sync();
    if (total) *total = ctx->host_scalars[0];
}

void merge_sorted(Ctx *ctx, const uint64_t *a, uint64_t na, const uint64_t *b, uint64_t nb, uint64_t *out) {
    merge_sorted_dev(ctx, a, na, nullptr, b, nb, nullptr, out, nullptr, nullptr);
}
void merge_sorted_dev(Ctx *ctx, const uint64_t *a, uint64_t na, const uint64_t *d_na, const uint64_t *b, uint64_t nb,
                      const uint64_t *d_nb, uint64_t *out, const uint64_t *skip, const uint32_t *stop) {
    uint64_t total = na + nb;
    if (!total) return;
    uint64_t tiles = (total + MRG_TILE - 1) / MRG_TILE;
    XH_REQUIRE(tiles < (1ull << 31), XLOG_HIP_CAPACITY_OVERFLOW, "merge: input too large");
    Buf<uint64_t> split(ctx, tiles + 1);
    MergeDev dv;
    dv.d_na = d_na;
    dv.d_nb = d_nb;
    dv.skip = skip;
    dv.stop = stop;
    hipLaunchKernelGGL(k_merge_partition, dim3((unsigned)((tiles + 1 + 255) / 256)), dim3(256), 0, ctx->stream, a, na,
                       b, nb, tiles, split.p, dv);
    XH_CHECK_HIP(hipGetLastError());
    // with device counts the bytes are counted on the device (work: 16 B per output row)
    const bool dev = d_na || d_nb;
    Prof prof(ctx, XLOG_HIP_KERNEL_MERGE, dev ? 0.0 : 16.0 * (double)total);
    if (dev) add_work_rows(ctx, prof.work(16.0), d_na, na, 1, d_nb, nb, 1, skip, stop);
    static const uint32_t merge_per_cu = [] {
        const char *e = getenv("XLOG_HIP_MERGE_PER_CU");
        const unsigned long v = e ? strtoul(e, nullptr, 10) : 0ul;
        return v ? (uint32_t)v : 32u;
    }();
    hipLaunchKernelGGL(k_merge, dim3(dev ? persistent_grid(ctx, tiles, merge_per_cu) : (unsigned)tiles), dim3(MRG_BLOCK), 0,
                       ctx->stream, a, na, b, nb, split.p, out, dv);
    XH_CHECK_HIP(hipGetLastError());
}

void pack_columns(Ctx *ctx, const uint32_t *c0, const uint32_t *c1, uint64_t n, uint64_t *out) {
    if (!n) return;
    hipLaunchKernelGGL(k_pack, dim3(grid_for(n, 256, 16384)), dim3(256), 0, ctx->stream, c0, c1, n, out);
    XH_CHECK_HIP(hipGetLastError());
}
void unpack_column(Ctx *ctx, const uint64_t *w, int hi, uint64_t n, uint32_t *out) {
    if (!n) return;
    hipLaunchKernelGGL(k_unpack, dim3(grid_for(n, 256, 16384)), dim3(256), 0, ctx->stream, w, hi, n, out);
    XH_CHECK_HIP(hipGetLastError());
}
void swap_words(Ctx *ctx, const uint64_t *in, uint64_t n, uint64_t *out) {
    if (!n) return;
    hipLaunchKernelGGL(k_swap, dim3(grid_for(n, 256, 16384)), dim3(256), 0, ctx->stream, in, n, out);
    XH_CHECK_HIP(hipGetLastError());
}
void low_words(Ctx *ctx, const uint64_t *in, uint64_t n, uint32_t *out) { unpack_column(ctx, in, 0, n, out); }

int is_sorted_u64(Ctx *ctx, const uint64_t *k, uint64_t n, int strict) {
    if (n < 2) return 1;
    Buf<uint32_t> flag(ctx, 2);
    fill_u32(ctx, flag.p, 0u, 1);
    hipLaunchKernelGGL(k_unsorted, dim3(grid_for(n, 256, 16384)), dim3(256), 0, ctx->stream, k, n, strict, flag.p);
    XH_CHECK_HIP(hipGetLastError());
    uint32_t h = 0;
    XH_CHECK_HIP(hipMemcpyAsync(&h, flag.p, sizeof(uint32_t), hipMemcpyDeviceToHost, ctx->stream));
    ctx->sync();
    return h == 0;
}

}  // namespace xh
