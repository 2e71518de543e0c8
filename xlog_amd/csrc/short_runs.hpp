// Placement step shared by the short-run sort kernels (sort.hip,
// k_sort_short_runs; select.hip, k_short_runs_unique).
//
// Input: keys sorted by their high word.  A run is a maximal range of keys
// with one high word; sorting every run by its low word (stably) sorts the
// keys in full.  A block owns the runs that start in its core
// [core_lo, core_lo + CORE) and loads the core, one key before it (to see
// whether the core's first key starts a run) and MAXR keys after it (a run
// that starts in the core ends there at the latest).  Each loaded key gets
// its run's start and end from a block-wide max-scan of run heads and
// min-scan of run tails; a key of an owned run then counts the run's keys
// that are smaller (an equal key counts as smaller when it comes earlier, so
// equal keys keep their order), and that count places it in the run.
#pragma once

#include "internal.hpp"

namespace xh {

template <int BLOCK, int CORE, int MAXR>
struct ShortRunTile {
    static constexpr int LEN = ((CORE + MAXR + 1 + BLOCK - 1) / BLOCK) * BLOCK;  // loaded keys, rounded up
    static constexpr int ITEMS = LEN / BLOCK;                                   // consecutive keys per thread
    uint32_t hi[LEN], lo[LEN];  // the loaded keys, then the placed keys (local index = place)
    uint32_t wmax[BLOCK / WAVE], wmin[BLOCK / WAVE];
    uint32_t pmin, pmax;  // the placed range [pmin, pmax)
};

// Loads the tile whose core starts at core_lo and places the keys of the runs
// it owns at their sorted position in t.hi / t.lo (local index, relative to
// the returned first loaded index).  On return (after a barrier) the placed
// keys fill [t.pmin, t.pmax) when no run is long; a run longer than MAXR keys
// sets *long_run and its keys are not placed.  Every thread of the block
// calls it.
template <int BLOCK, int CORE, int MAXR>
__device__ __forceinline__ uint64_t short_runs_place(const uint64_t *__restrict__ in, uint64_t n, uint64_t core_lo,
                                                     ShortRunTile<BLOCK, CORE, MAXR> &t, uint64_t *long_run) {
    using T = ShortRunTile<BLOCK, CORE, MAXR>;
    constexpr int ITEMS = T::ITEMS;
    constexpr uint32_t NONE = 0xFFFFFFFFu;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    if (tid == 0) {
        t.pmin = NONE;
        t.pmax = 0;
    }
    const uint64_t core_hi = core_lo + CORE < n ? core_lo + CORE : n;
    const uint64_t lo = core_lo > 0 ? core_lo - 1 : 0;
    const uint64_t hi = core_hi + MAXR < n ? core_hi + MAXR : n;
    const uint32_t len = (uint32_t)(hi - lo);
    batched_copy<BLOCK, ITEMS>(
        len, tid, [&](uint32_t i) { return in[lo + i]; },
        [&](uint32_t i, uint64_t k) {
            t.hi[i] = (uint32_t)(k >> 32);
            t.lo[i] = (uint32_t)k;
        });
    __syncthreads();
    // thread `tid` owns ITEMS consecutive keys: run start = last head at or
    // before the key, run end = first tail at or after it, plus one (the
    // first loaded key counts as a head: a run through it starts before the
    // core and is not owned)
    const uint32_t b0 = (uint32_t)tid * ITEMS;
    uint32_t hv[ITEMS + 2];
#pragma unroll
    for (int q = -1; q <= ITEMS; ++q) {
        const int i = (int)b0 + q;
        hv[q + 1] = (i >= 0 && i < (int)len) ? t.hi[i] : 0u;
    }
    uint32_t hmax = 0, tmin = NONE;
    uint32_t st_loc[ITEMS], en_loc[ITEMS];
#pragma unroll
    for (int q = 0; q < ITEMS; ++q) {
        const uint32_t i = b0 + q;
        if (i < len && (i == 0 || hv[q + 1] != hv[q])) hmax = i;
        st_loc[q] = hmax;
    }
#pragma unroll
    for (int q = ITEMS - 1; q >= 0; --q) {
        const uint32_t i = b0 + q;
        if (i < len && (i + 1 == len || hv[q + 1] != hv[q + 2])) tmin = i + 1;
        en_loc[q] = tmin;
    }
    // exclusive max-scan of the threads' last heads and min-scan (from the
    // right) of their first tails over the block
    uint32_t incl_max = hmax, incl_min = tmin;
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
        const uint32_t a = __shfl_up(incl_max, o, WAVE);
        const uint32_t c = __shfl_down(incl_min, o, WAVE);
        if (lane >= o) incl_max = a > incl_max ? a : incl_max;
        if (lane + o < WAVE) incl_min = c < incl_min ? c : incl_min;
    }
    if (lane == WAVE - 1) t.wmax[wave] = incl_max;
    if (lane == 0) t.wmin[wave] = incl_min;
    __syncthreads();
    uint32_t before = __shfl_up(incl_max, 1, WAVE), after = __shfl_down(incl_min, 1, WAVE);
    if (lane == 0) before = 0;
    if (lane == WAVE - 1) after = NONE;
#pragma unroll
    for (int w = 0; w < BLOCK / WAVE; ++w) {
        if (w < wave) before = t.wmax[w] > before ? t.wmax[w] : before;
        if (w > wave) after = t.wmin[w] < after ? t.wmin[w] : after;
    }
    bool longr = false;
    uint32_t klo[ITEMS], place[ITEMS];
#pragma unroll
    for (int q = 0; q < ITEMS; ++q) {
        const uint32_t li = b0 + q;
        place[q] = NONE;
        klo[q] = 0;
        if (li >= len || lo + li < core_lo) continue;
        const uint32_t st = st_loc[q] > before ? st_loc[q] : before;
        const uint32_t e = en_loc[q] < after ? en_loc[q] : after;
        if (e - st > (uint32_t)MAXR) {  // a run of more than MAXR keys
            longr = true;
            continue;
        }
        // runs that start before the core or after it belong to other blocks
        if (lo + st < core_lo || lo + st >= core_hi) continue;
        if (e == len && hi < n && (uint32_t)(in[hi] >> 32) == hv[q + 1]) {  // continues past the loaded keys
            longr = true;
            continue;
        }
        const uint32_t my = t.lo[li];
        uint32_t r = 0;
        if (e - st > 1) {
            // the run shares the high word, so (low word, position) orders it:
            // one 64-bit compare per key of the run, four loads in flight
            const uint64_t mine = ((uint64_t)my << 32) | li;
            uint32_t j = st;
            for (; j + 4 <= e; j += 4) {
                uint32_t cj[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) cj[u] = t.lo[j + u];
#pragma unroll
                for (int u = 0; u < 4; ++u) r += ((((uint64_t)cj[u] << 32) | (j + u)) < mine) ? 1u : 0u;
            }
            for (; j < e; ++j) r += ((((uint64_t)t.lo[j] << 32) | j) < mine) ? 1u : 0u;
        }
        klo[q] = my;
        place[q] = st + r;
    }
    if (__ballot(longr) != 0 && lane == 0) *long_run = 1ull;
    __syncthreads();  // every rank has read t.lo: the arrays now take the placed keys
    uint32_t pmin = NONE, pmax = 0;
#pragma unroll
    for (int q = 0; q < ITEMS; ++q) {
        if (place[q] == NONE) continue;
        t.hi[place[q]] = hv[q + 1];
        t.lo[place[q]] = klo[q];
        pmin = place[q] < pmin ? place[q] : pmin;
        pmax = place[q] + 1 > pmax ? place[q] + 1 : pmax;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint32_t a = __shfl_xor(pmin, o, WAVE), c = __shfl_xor(pmax, o, WAVE);
        pmin = a < pmin ? a : pmin;
        pmax = c > pmax ? c : pmax;
    }
    if (lane == 0 && pmin != NONE) {
        atomicMin(&t.pmin, pmin);
        atomicMax(&t.pmax, pmax);
    }
    __syncthreads();
    return lo;
}

}  // namespace xh
