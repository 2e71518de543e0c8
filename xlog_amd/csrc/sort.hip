// LSD radix sort of packed u64 tuple keys for gfx950.
//
// Replaces the reference's 4-bit, 8-passes-per-u32-column sort
// (crates/xlog-cuda/src/provider/relational.rs:1881-2357, kernels/sort.cu:28-264)
// with a onesweep design:
//   1. k_hist8: one read of the keys builds the 256-bin histograms of the
//      digits the sort uses (all eight for a full-key sort; a large full-key
//      sort counts the high word's four first and the low word's with a second
//      read only when it takes a pass over a low digit); a digit above
//      the lowest whose histogram has a single non-empty bin is constant over
//      the input and its pass is skipped (the lowest digit's pass is queued
//      before the histograms reach the host, so it always runs).
//   2. k_onesweep, once per remaining digit: a tile of TILE keys is ranked
//      per wave with 64-lane ballot matching (stable), the tile's 256 digit
//      counts are published and the exclusive prefix over earlier tiles is
//      obtained by decoupled look-back, the tile is reordered by digit in
//      LDS and written out so that consecutive lanes write consecutive
//      addresses of a digit run.
//   3. For a large keys-only sort of the whole key whose high word leaves
//      runs of a few keys (estimated from the histograms), only the high
//      word's digits take passes; k_sort_short_runs then orders every run of
//      equal high word by its low word in one more pass (4 + 1 passes over
//      uniform keys instead of 8).
// Each pass reads and writes every key exactly once (16 B per key, plus the
// optional u32 payload).  Tiles go to the XCDs in chunks of consecutive
// tiles, so that neighbouring tiles share an L2, and a tile only ever waits
// for tiles of earlier-dispatched blocks.
#include "internal.hpp"
#include "short_runs.hpp"

#include <atomic>

namespace xh {

namespace {

// Tile shapes: BLOCK threads (>= 256; threads 0..255 own one digit each in
// the counting phase) x ITEMS keys per thread.  512x16 (8192 keys, 74 KB LDS,
// 2 blocks per CU); key + payload sorts need LDS for the payload too, hence
// a smaller tile.
#ifndef XH_SORT_BLOCK_K
#define XH_SORT_BLOCK_K 512
#endif
#ifndef XH_SORT_ITEMS_K
#define XH_SORT_ITEMS_K 16
#endif
#ifndef XH_SORT_BLOCK_V
#define XH_SORT_BLOCK_V 256
#endif
#ifndef XH_SORT_ITEMS_V
#define XH_SORT_ITEMS_V 16
#endif
#ifndef XH_SORT_LOOKBACK
#define XH_SORT_LOOKBACK 4
#endif
constexpr int SORT_LOOKBACK = XH_SORT_LOOKBACK;

constexpr int SORT_BLOCK_K = XH_SORT_BLOCK_K, SORT_ITEMS_K = XH_SORT_ITEMS_K;
constexpr int SORT_BLOCK_V = XH_SORT_BLOCK_V, SORT_ITEMS_V = XH_SORT_ITEMS_V;
static_assert(SORT_BLOCK_K >= 256 && SORT_BLOCK_K % 256 == 0 && SORT_BLOCK_V >= 256 && SORT_BLOCK_V % 256 == 0,
              "digit phase needs 256 threads");
constexpr uint32_t ST_AGG = 1u << 30;
constexpr uint32_t ST_INC = 2u << 30;
constexpr uint32_t ST_VAL = (1u << 30) - 1;

__device__ __forceinline__ uint32_t ld_status(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_status(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Histograms of the digits [dlo, dhi) in one read of the keys.  A block of
// HIST_BLOCK threads reads HIST_ITEMS keys per thread per round, coalesced
// (key base + r * HIST_BLOCK + tid), with the next round's loads in flight,
// and adds every counted digit to LDS counters held in HIST_COPIES interleaved
// copies (lane l adds to copy l % HIST_COPIES), so that the random bins of one
// instruction's lanes spread over more LDS banks: bank conflicts, not the
// loads, bound a single-copy histogram of random keys (measured on MI355X over
// 2^28 random keys: 0.54 ms with one copy, 0.47-0.51 ms with four; a plain
// read of the keys takes 0.30 ms).  A digit that has one value in all of a
// wave's keys of the round (the constant digits of a narrow domain, the high
// words of a run of equal keys) is added once by the wave's first lane
// instead of by every lane on one counter.
constexpr int HIST_BLOCK = 512, HIST_ITEMS = 8, HIST_COPIES = 4;
__global__ __launch_bounds__(HIST_BLOCK) void k_hist8(const uint64_t *__restrict__ keys, uint64_t n,
                                                      uint32_t *__restrict__ ghist, int dlo, int dhi,
                                                      const uint64_t *d_n, const uint32_t *stop) {
    __shared__ uint32_t h[8 * 256 * HIST_COPIES];
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    // queued iterations: the key count on the device (n is its bound) and the stop flag
    if (stop && *stop) return;
    if (d_n && *d_n < n) n = *d_n;
    for (int i = tid; i < 8 * 256 * HIST_COPIES; i += HIST_BLOCK) h[i] = 0;
    __syncthreads();
    uint32_t *hs = h + (lane % HIST_COPIES);
    const uint32_t counted = (0xFFu >> (8 - dhi)) & ~((1u << dlo) - 1u);  // digits [dlo, dhi)
    const uint64_t round = (uint64_t)HIST_BLOCK * HIST_ITEMS, gstride = (uint64_t)gridDim.x * round;
    uint64_t pre[HIST_ITEMS];
    uint64_t t0 = (uint64_t)blockIdx.x * round;
#pragma unroll
    for (int r = 0; r < HIST_ITEMS; ++r) {
        const uint64_t j = t0 + (uint64_t)r * HIST_BLOCK + tid;
        pre[r] = j < n ? __builtin_nontemporal_load(keys + j) : 0ull;
    }
    for (; t0 < n; t0 += gstride) {
        uint64_t k[HIST_ITEMS];
#pragma unroll
        for (int r = 0; r < HIST_ITEMS; ++r) k[r] = pre[r];
        const uint64_t t1 = t0 + gstride;
#pragma unroll
        for (int r = 0; r < HIST_ITEMS; ++r) {
            const uint64_t j = t1 + (uint64_t)r * HIST_BLOCK + tid;
            pre[r] = j < n ? __builtin_nontemporal_load(keys + j) : 0ull;
        }
        // the wave's valid keys in this round (scalar) and the digits on which
        // some valid key differs from the first lane's first key
        const uint64_t wb = t0 + (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane(wave) * WAVE;
        uint32_t wtot = 0;
#pragma unroll
        for (int r = 0; r < HIST_ITEMS; ++r) {
            const uint64_t b = wb + (uint64_t)r * HIST_BLOCK;
            wtot += b >= n ? 0u : (n - b >= (uint64_t)WAVE ? (uint32_t)WAVE : (uint32_t)(n - b));
        }
        if (wtot == 0) continue;  // wave-uniform: past the end
        const uint64_t k0 = (uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)k[0]) |
                            ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(k[0] >> 32)) << 32);
        uint64_t x = 0;
#pragma unroll
        for (int r = 0; r < HIST_ITEMS; ++r) {
            const uint64_t j = t0 + (uint64_t)r * HIST_BLOCK + tid;
            x |= j < n ? k[r] ^ k0 : 0ull;
        }
        uint32_t varying = 0;
#pragma unroll
        for (int d = 0; d < 8; ++d) varying |= (__ballot(((x >> (8 * d)) & 255u) != 0) ? 1u : 0u) << d;
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            if (!((counted >> d) & 1u)) continue;
            if (!((varying >> d) & 1u)) {
                if (lane == 0) atomicAdd(&hs[(d * 256 + (uint32_t)((k0 >> (8 * d)) & 255u)) * HIST_COPIES], wtot);
                continue;
            }
#pragma unroll
            for (int r = 0; r < HIST_ITEMS; ++r) {
                const uint64_t j = t0 + (uint64_t)r * HIST_BLOCK + tid;
                if (j < n) atomicAdd(&hs[(d * 256 + (uint32_t)((k[r] >> (8 * d)) & 255u)) * HIST_COPIES], 1u);
            }
        }
    }
    __syncthreads();
    for (int i = tid; i < 8 * 256; i += HIST_BLOCK) {
        if (!((counted >> (i >> 8)) & 1u)) continue;
        uint32_t c = 0;
#pragma unroll
        for (int q = 0; q < HIST_COPIES; ++q) c += h[i * HIST_COPIES + q];
        if (c) atomicAdd(&ghist[i], c);
    }
}

// exclusive scan of each of the 8 histograms -> offsets[8][256]
__global__ void k_digit_offsets(const uint32_t *__restrict__ ghist, uint32_t *__restrict__ off) {
    int d = threadIdx.x;
    if (d < 8) {
        uint32_t acc = 0;
        for (int b = 0; b < 256; ++b) {
            uint32_t c = ghist[d * 256 + b];
            off[d * 256 + b] = acc;
            acc += c;
        }
    }
}

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v, int lane) {
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
        uint32_t t = __shfl_up(v, o, WAVE);
        if (lane >= o) v += t;
    }
    return v;
}

// Tile order of the digit passes.  Consecutive tiles write adjacent pieces of
// every digit run, so their partial cache lines merge only when they run under
// one L2.  Workgroups are dispatched in index order, round-robin over the 8
// XCDs, so tiles go out in chunks of `chunk` consecutive tiles: block b runs
// tile ((j / chunk) * 8 + b % 8) * chunk + j % chunk with j = b / 8, i.e. chunk
// k goes to the blocks with b % 8 == k % 8 (one XCD).  Within each group of
// 8 * chunk blocks this is a permutation, and a tile waits only on tiles of
// its own or earlier groups.  The look-back therefore always ends under two
// conditions: (1) workgroups start in index order, and (2) the device holds at
// least 8 * chunk blocks of the pass at once (the host sizes chunk to 1/16 of
// what it holds).  If either failed, a tile could wait on a tile whose block
// cannot start, and the pass would never finish.  The ticketed order
// (XLOG_HIP_SORT_TICKETS=1) numbers blocks by an atomic ticket taken at start
// instead of their index, which removes condition (1) and keeps (2).  Measured
// on MI355X: chunked by index 1.07 ms per 2^28-key pass (0.081 ms at 2^24),
// chunked by ticket 1.21 ms (blocks start in a slightly different order on
// each XCD, which breaks the chunk-to-XCD placement), plain ticket order 1.16 ms.
constexpr uint32_t TILE_NONE = 0xFFFFFFFFu;

__device__ __forceinline__ uint32_t chunk_tile(uint32_t b, uint32_t chunk, uint32_t tiles) {
    const uint32_t q = b & 7u, j = b >> 3;
    const uint64_t t = ((uint64_t)(j / chunk) * 8 + q) * chunk + j % chunk;
    return t < tiles ? (uint32_t)t : TILE_NONE;
}

// The keys of tile j with digit d: the count tile j publishes, computed by a
// waiting tile instead (the bounded wait of the look-back, below).
__device__ uint32_t tile_digit_count(const uint64_t *__restrict__ kin, uint64_t n, uint64_t j, uint64_t tile_keys,
                                     int shift, uint32_t d) {
    const uint64_t a = j * tile_keys, b = a + tile_keys < n ? a + tile_keys : n;
    uint32_t c = 0;
    for (uint64_t i = a; i < b; ++i) c += (((uint32_t)(kin[i] >> shift) & 255u) == d) ? 1u : 0u;
    return c;
}

// The look-back's wait is bounded: a digit thread that finds the tile before
// the ones it has consumed unpublished for spin_limit polls in a row counts
// that tile's keys of its digit itself (they are in kin before the pass
// starts) and walks on.  Its prefix is the one the tile would have published,
// so the pass needs no assumption on dispatch order or residency: a tile
// whose predecessor's block has not started (out-of-order dispatch, or fewer
// co-resident blocks than a chunk group) only costs the waiting tile a read
// of that predecessor, and under in-order dispatch the bound is never reached.
template <bool HAS_VAL, int BLOCK, int ITEMS>
__global__ __launch_bounds__(BLOCK) void k_onesweep(
    const uint64_t *__restrict__ kin, uint64_t *__restrict__ kout, const uint32_t *__restrict__ vin,
    uint32_t *__restrict__ vout, uint64_t n, uint32_t tiles, int shift, const uint32_t *__restrict__ digit_off,
    uint32_t *status, uint32_t *status_next, uint32_t chunk, unsigned long long *ticket,
    unsigned long long ticket_base, const uint64_t *d_n, const uint32_t *stop, uint32_t spin_limit) {
    __shared__ uint32_t s_wcnt[(BLOCK / WAVE)][256];
    __shared__ uint32_t s_ticket;
    __shared__ uint32_t s_gbase[256];
    __shared__ uint32_t s_wsum[(BLOCK / WAVE)];
    __shared__ uint64_t s_keys[(BLOCK * ITEMS)];
    __shared__ uint32_t s_vals[HAS_VAL ? (BLOCK * ITEMS) : 1];

    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    const uint32_t lane_u = (uint32_t)lane;
    const int d = tid;
    const bool digit_thread = tid < 256;
    // The tile comes from the block index (default: tiles stay on their XCD
    // under in-order dispatch) or, in the ticketed order, from the block's
    // start-order ticket, so that a tile only ever waits on tiles of blocks that
    // started before it or belong to its own group of 8 * chunk tickets,
    // whatever order the blocks are dispatched in.  Block-uniform, so it (and
    // every per-round bound derived from it) stays in scalar registers.
    // A key count on the device (d_n: a queued iteration's sort; n and tiles
    // are then bounds) makes the pass persistent: a grid of at most the blocks
    // the device holds takes tickets in plain order from a counter zeroed for
    // the pass (ticket_base 0) until they pass the tiles that hold keys, so a
    // tile waits only on tiles whose blocks took their tickets before it.  A
    // stop raised by an earlier launch of the queue ends every block.
    const bool persist = d_n != nullptr;
    uint32_t real_tiles = tiles;
    if (persist) {
        if (stop && *stop) return;
        if (*d_n < n) n = *d_n;
        real_tiles = (uint32_t)((n + (uint64_t)(BLOCK * ITEMS) - 1) / (uint64_t)(BLOCK * ITEMS));
        if (blockIdx.x >= real_tiles) return;  // more blocks than tiles: these take no ticket
    }
    for (;;) {
    if (ticket && tid == 0) s_ticket = (uint32_t)(atomicAdd(ticket, 1ull) - ticket_base);
    for (int i = tid; i < (BLOCK / WAVE) * 256; i += BLOCK) (&s_wcnt[0][0])[i] = 0;
    __syncthreads();
    const uint32_t tile = persist ? __builtin_amdgcn_readfirstlane(s_ticket)
                                  : chunk_tile(ticket ? __builtin_amdgcn_readfirstlane(s_ticket) : blockIdx.x, chunk,
                                               tiles);
    if (tile == TILE_NONE || tile >= real_tiles) {
        if (persist && tid == 0) persist_done(ticket, gridDim.x < real_tiles ? gridDim.x : real_tiles);
        return;
    }
    {  // one tile
        const uint64_t wbase =
            (uint64_t)tile * (BLOCK * ITEMS) + (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane(wave) * (ITEMS * WAVE);
        // valid keys of this wave (0..ITEMS*WAVE) and of its round r (0..64)
        const int32_t wleft =
            wbase >= n ? 0 : ((n - wbase) >= (uint64_t)(ITEMS * WAVE) ? ITEMS * WAVE : (int32_t)(n - wbase));
        auto round_valid = [&](int r) -> uint32_t {
            const int32_t rem = wleft - r * WAVE;
            return rem <= 0 ? 0u : (rem >= WAVE ? (uint32_t)WAVE : (uint32_t)rem);
        };

        uint64_t k[ITEMS];
        uint32_t v[ITEMS];
        uint32_t rank[ITEMS];
#pragma unroll
        for (int r = 0; r < ITEMS; ++r) {
            const uint64_t idx = wbase + (uint64_t)r * WAVE + lane;
            const bool valid = (uint32_t)lane < round_valid(r);
            k[r] = valid ? kin[idx] : 0ull;
            if (HAS_VAL) v[r] = valid ? vin[idx] : 0u;
        }
        // Stable rank of each key among the wave's keys of equal digit, two
        // rounds at a time so that the two ballot chains interleave.  A lane's
        // peers are the lanes whose 8 digit bits all agree with its own; the
        // lanes that disagree on bit b are ballot(bit b) ^ splat(own bit b),
        // accumulated over the 8 bits as a mismatch mask (invalid lanes start
        // mismatched).
        static_assert(ITEMS % 2 == 0, "rounds are ranked in pairs");
#pragma unroll
        for (int r = 0; r < ITEMS; r += 2) {
            uint32_t dg[2], mlo[2], mhi[2], nv[2];
#pragma unroll
            for (int qq = 0; qq < 2; ++qq) {
                dg[qq] = (uint32_t)(k[r + qq] >> shift) & 255u;
                nv[qq] = round_valid(r + qq);
                const uint64_t vm = nv[qq] >= (uint32_t)WAVE ? ~0ull : ((1ull << nv[qq]) - 1ull);
                mlo[qq] = ~(uint32_t)vm;
                mhi[qq] = ~(uint32_t)(vm >> 32);
            }
#pragma unroll
            for (int b = 0; b < 8; ++b) {
#pragma unroll
                for (int qq = 0; qq < 2; ++qq) {
                    // s = 0 or ~0: bit b of the digit, sign-extended.  The empty
                    // asm keeps the ballot's compare on s itself (v_bfe + v_cmp)
                    // instead of a recomputed shift of the digit.
                    uint32_t s = (uint32_t)__builtin_amdgcn_sbfe((int32_t)dg[qq], b, 1);
                    asm("" : "+v"(s));
                    const uint64_t m = __ballot(s != 0u);
                    mlo[qq] |= (uint32_t)m ^ s;
                    mhi[qq] |= (uint32_t)(m >> 32) ^ s;
                }
            }
#pragma unroll
            for (int qq = 0; qq < 2; ++qq) {
                // peers below = lanes below - mismatched lanes below
                const uint32_t below =
                    lane_u - __builtin_amdgcn_mbcnt_hi(mhi[qq], __builtin_amdgcn_mbcnt_lo(mlo[qq], 0u));
                // every peer reads the running count before the group's first
                // lane bumps it: LDS operations of one wave complete in order
                const uint32_t old = s_wcnt[wave][dg[qq]];
                if (below == 0 && lane_u < nv[qq])
                    s_wcnt[wave][dg[qq]] = old + (uint32_t)WAVE - (uint32_t)(__popc(mlo[qq]) + __popc(mhi[qq]));
                rank[r + qq] = old + below;
            }
        }
        __syncthreads();

        // per digit (threads 0..255): totals and exclusive prefix over waves
        uint32_t cnt = 0, incl = 0;
        uint32_t *my = status + (uint64_t)tile * 256 + d;
        if (digit_thread) {
#pragma unroll
            for (int w = 0; w < (BLOCK / WAVE); ++w) {
                uint32_t c = s_wcnt[w][d];
                s_wcnt[w][d] = cnt;
                cnt += c;
            }
            // publish this tile's aggregate (or inclusive prefix for tile 0)
            st_status(my, (tile == 0 ? ST_INC : ST_AGG) | cnt);
            // tile-local exclusive scan over the 256 digits (waves 0..3)
            incl = wave_incl_scan(cnt, lane);
            if (lane == WAVE - 1) s_wsum[wave] = incl;
        }
        __syncthreads();
        if (digit_thread) {
            uint32_t wpre = 0;
#pragma unroll
            for (int w = 0; w < 4; ++w)
                if (w < wave) wpre += s_wsum[w];
            const uint32_t tstart = wpre + incl - cnt;
            // fold the digit's tile start into the per-wave bases: the reorder
            // then reads one LDS word per key instead of two
#pragma unroll
            for (int w = 0; w < (BLOCK / WAVE); ++w) s_wcnt[w][d] += tstart;
            s_gbase[d] = tstart;  // parked until the look-back below replaces it
        }
        __syncthreads();

        // reorder the tile by digit in LDS: positions inside the tile do not
        // depend on earlier tiles, so this comes before the look-back, frees
        // the key registers during it and overlaps it with the other waves'
        // LDS writes (with the chunked tile order: 1.19 -> 1.07 ms per
        // 2^28-key pass)
#pragma unroll
        for (int r = 0; r < ITEMS; ++r) {
            if ((uint32_t)lane < round_valid(r)) {
                const uint32_t dd = (uint32_t)(k[r] >> shift) & 255u;
                const uint32_t pos = s_wcnt[wave][dd] + rank[r];
                s_keys[pos] = k[r];
                if (HAS_VAL) s_vals[pos] = v[r];
            }
        }
        if (digit_thread) {
            const uint32_t tstart = s_gbase[d];
            // decoupled look-back over earlier tiles for this digit
            // (SORT_LOOKBACK predecessors are loaded at once; the walk consumes
            // them in order and resumes at the first one not yet published;
            // wider or growing batches measured slower)
            uint32_t prefix = 0;
            if (tile > 0) {
                int64_t j = (int64_t)tile - 1;
                bool done = false;
                uint32_t spins = 0;
                while (!done) {
                    uint32_t st[SORT_LOOKBACK];
#pragma unroll
                    for (int z = 0; z < SORT_LOOKBACK; ++z)
                        // tile 0 is inclusive, so the walk never passes it; the
                        // guard only keeps the batch's loads in bounds
                        st[z] = j - z >= 0 ? ld_status(status + (uint64_t)(j - z) * 256 + d) : ST_INC;
                    // consume the published prefix of the batch, up to and
                    // including the first inclusive entry (branch-free)
                    uint32_t pub = 0, inc = 0;
#pragma unroll
                    for (int z = 0; z < SORT_LOOKBACK; ++z) {
                        const uint32_t flag = st[z] & ~ST_VAL;
                        pub |= (flag != 0u ? 1u : 0u) << z;
                        inc |= (flag == ST_INC ? 1u : 0u) << z;
                    }
                    const int first_unpub = __builtin_ctz(~pub);
                    const int first_inc = inc ? __builtin_ctz(inc) : 32;
                    done = first_inc < first_unpub;
                    const int used = done ? first_inc + 1 : first_unpub;
#pragma unroll
                    for (int z = 0; z < SORT_LOOKBACK; ++z) prefix += z < used ? (st[z] & ST_VAL) : 0u;
                    j -= used;
                    if (used > 0) {
                        spins = 0;
                    } else if (++spins > spin_limit) {  // tile j has not published: count it here
                        prefix += tile_digit_count(kin, n, (uint64_t)j, (uint64_t)(BLOCK * ITEMS), shift, (uint32_t)d);
                        j -= 1;
                        spins = 0;
                        done = j < 0;
                    }
                }
                st_status(my, ST_INC | (prefix + cnt));
            }
            s_gbase[d] = digit_off[d] + prefix - tstart;
            // the next pass uses the other status buffer: clear this tile's slot there
            status_next[(uint64_t)tile * 256 + d] = 0u;
        }
        __syncthreads();
        const uint64_t t0 = (uint64_t)tile * (BLOCK * ITEMS);
        const uint32_t tn = (uint32_t)((n - t0) < (uint64_t)(BLOCK * ITEMS) ? (n - t0) : (uint64_t)(BLOCK * ITEMS));
        for (uint32_t i = tid; i < tn; i += BLOCK) {
            const uint64_t key = s_keys[i];
            const uint32_t dd = (uint32_t)(key >> shift) & 255u;
            const uint64_t o = (uint64_t)s_gbase[dd] + i;
            if (o < n) {  // always true for a consistent histogram; keeps a bad one in bounds
                kout[o] = key;
                if (HAS_VAL) vout[o] = s_vals[i];
            }
        }
    }
    if (!persist) return;
    __syncthreads();  // the shared arrays are reused by the next tile
    }
}

// Sort of short runs: keys sorted by their high word, each run of equal high
// word sorted by its low word in place of the low word's radix passes (the
// placement is short_runs_place).  The placed keys sit in LDS at their place
// and the block's range of places (its runs are contiguous) is written out in
// one coalesced sweep.  A run longer than SR_MAX keys sets *long_run (its keys
// are then not placed and the caller sorts the whole input instead).
constexpr int SR_BLOCK = 256, SR_CORE = 2048, SR_MAX = 256;
using SrTile = ShortRunTile<SR_BLOCK, SR_CORE, SR_MAX>;
__global__ __launch_bounds__(SR_BLOCK) void k_sort_short_runs(const uint64_t *__restrict__ in, uint64_t n,
                                                              uint64_t *__restrict__ out, uint64_t *long_run) {
    __shared__ SrTile t;
    const uint64_t lo = short_runs_place<SR_BLOCK, SR_CORE, SR_MAX>(in, n, (uint64_t)blockIdx.x * SR_CORE, t, long_run);
    for (uint32_t i = t.pmin + threadIdx.x; i < t.pmax; i += SR_BLOCK) out[lo + i] = ((uint64_t)t.hi[i] << 32) | t.lo[i];
}
// The same over a key count on the device (n is its bound): a grid of a few
// blocks per CU strides over the cores; nothing when *stop is raised.
__global__ __launch_bounds__(SR_BLOCK) void k_sort_short_runs_dev(const uint64_t *__restrict__ in, uint64_t n,
                                                                  const uint64_t *d_n, uint64_t *__restrict__ out,
                                                                  uint64_t *long_run, const uint32_t *stop) {
    __shared__ SrTile t;
    if (stop && *stop) return;
    if (*d_n < n) n = *d_n;
    for (uint64_t core = (uint64_t)blockIdx.x * SR_CORE; core < n; core += (uint64_t)gridDim.x * SR_CORE) {
        const uint64_t lo = short_runs_place<SR_BLOCK, SR_CORE, SR_MAX>(in, n, core, t, long_run);
        for (uint32_t i = t.pmin + threadIdx.x; i < t.pmax; i += SR_BLOCK)
            out[lo + i] = ((uint64_t)t.hi[i] << 32) | t.lo[i];
        __syncthreads();  // t is reused by the next core
    }
}
// skip = 1 unless the short-run pass found a long run (and the queue runs)
__global__ void k_fallback_skip(const uint64_t *long_run, const uint32_t *stop, uint32_t *skip) {
    *skip = ((stop && *stop) || *long_run == 0) ? 1u : 0u;
}
__global__ void k_copy_dev(const uint64_t *__restrict__ in, uint64_t n, const uint64_t *d_n, uint64_t *__restrict__ out,
                           const uint32_t *skip) {
    if (*skip) return;
    if (*d_n < n) n = *d_n;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = in[i];
}

__global__ void k_fill_u32(uint32_t *p, uint32_t v, uint64_t n) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}
__global__ void k_fill_u64(uint64_t *p, uint64_t v, uint64_t n) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

// Zero-fill of several u64 ranges in one launch: range blockIdx.y, grid-stride
// over its words (blocks past a short range's end exit at once).
struct FillRangesArgs {
    uint64_t *p[FILL_MAX_RANGES];
    uint64_t n[FILL_MAX_RANGES];
};
__global__ void k_fill_ranges(FillRangesArgs a) {
    uint64_t *p = a.p[blockIdx.y];
    const uint64_t n = a.n[blockIdx.y], stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0ull;
}

}  // namespace

void FillBatch::flush() {
    for (size_t b = 0; b < r.size(); b += FILL_MAX_RANGES) {
        FillRangesArgs a{};
        const size_t k = std::min<size_t>(FILL_MAX_RANGES, r.size() - b);
        uint64_t most = 0;
        for (size_t j = 0; j < k; ++j) {
            a.p[j] = r[b + j].first;
            a.n[j] = r[b + j].second;
            most = std::max(most, a.n[j]);
        }
        hipLaunchKernelGGL(k_fill_ranges, dim3(grid_for(most, 256, 4096), (unsigned)k), dim3(256), 0, ctx->stream, a);
        XH_CHECK_HIP(hipGetLastError());
    }
    r.clear();
}

void fill_u64(Ctx *ctx, uint64_t *p, uint64_t v, uint64_t n) {
    if (!n) return;
    hipLaunchKernelGGL(k_fill_u64, dim3(grid_for(n, 256, 8192)), dim3(256), 0, ctx->stream, p, v, n);
    XH_CHECK_HIP(hipGetLastError());
}
void fill_u32(Ctx *ctx, uint32_t *p, uint32_t v, uint64_t n) {
    if (!n) return;
    hipLaunchKernelGGL(k_fill_u32, dim3(grid_for(n, 256, 8192)), dim3(256), 0, ctx->stream, p, v, n);
    XH_CHECK_HIP(hipGetLastError());
}

// Look-back status buffers for the sort passes, kept per context.  Invariant
// tracked on the host: dirty[b] = number of leading tiles of buffer b that may
// hold non-zero entries.
struct SortState {
    uint32_t *status[2] = {nullptr, nullptr};
    uint64_t tiles_cap = 0;
    uint64_t dirty[2] = {0, 0};
    uint32_t *hist = nullptr;  // 8*256 counts + 8*256 offsets
};
static std::map<Ctx *, SortState> g_sort_state;
static std::mutex g_sort_mu;

void sort_state_release(Ctx *ctx) {
    std::lock_guard<std::mutex> g(g_sort_mu);
    auto it = g_sort_state.find(ctx);
    if (it == g_sort_state.end()) return;
    if (it->second.status[0]) ctx->free(it->second.status[0]);
    if (it->second.status[1]) ctx->free(it->second.status[1]);
    if (it->second.hist) ctx->free(it->second.hist);
    g_sort_state.erase(it);
}

static SortState &sort_state(Ctx *ctx, uint64_t tiles) {
    std::lock_guard<std::mutex> g(g_sort_mu);
    SortState &st = g_sort_state[ctx];
    if (!st.hist) st.hist = static_cast<uint32_t *>(ctx->alloc(2 * 8 * 256 * sizeof(uint32_t)));
    if (tiles > st.tiles_cap) {
        uint64_t cap = tiles < 1024 ? 1024 : tiles + tiles / 4;
        for (int b = 0; b < 2; ++b) {
            if (st.status[b]) ctx->free(st.status[b]);
            st.status[b] = static_cast<uint32_t *>(ctx->alloc(cap * 256 * sizeof(uint32_t)));
            fill_u32(ctx, st.status[b], 0u, cap * 256);
            st.dirty[b] = 0;
        }
        st.tiles_cap = cap;
    }
    return st;
}

// Blocks of one digit pass kernel that the device holds at once (occupancy
// queried once per process): the tile order needs 8 * chunk of them.
template <bool HAS_VAL, int BLOCK, int ITEMS>
static uint32_t pass_capacity(Ctx *ctx) {
    static std::atomic<int> per_cu{0};  // contexts on other threads may ask at the same time
    int b = per_cu.load(std::memory_order_relaxed);
    if (b == 0) {
        XH_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &b, reinterpret_cast<const void *>(&k_onesweep<HAS_VAL, BLOCK, ITEMS>), BLOCK, 0));
        if (b <= 0) b = 1;
        per_cu.store(b, std::memory_order_relaxed);
    }
    return (uint32_t)ctx->num_cus * (uint32_t)b;
}

// Tile order.  The digit passes take tiles by workgroup index in XCD chunks
// (chunk_tile) with the bounded look-back wait of k_onesweep, which keeps them
// correct whatever the dispatch order; XLOG_HIP_SORT_TICKETS=1 numbers their
// tiles by start tickets instead (plain order, 9-11 % slower per pass).  The
// fused short-run unique has no such fallback and takes start tickets unless
// XLOG_HIP_SORT_TICKETS=0 (workgroup-index order: correct only when the
// workgroups of a launch start in index order).
static int sort_tickets_env() {
    const char *e = getenv("XLOG_HIP_SORT_TICKETS");
    return e && (e[0] == '0' || e[0] == '1') ? e[0] - '0' : -1;
}
bool sort_tickets() { return sort_tickets_env() != 0; }
static bool pass_tickets() { return sort_tickets_env() == 1; }
// polls of an unpublished predecessor before a digit thread counts it itself
// (XLOG_HIP_SORT_SPIN; the tests set 0 to take the fallback at every wait)
static uint32_t sort_spin_limit() {
    const char *e = getenv("XLOG_HIP_SORT_SPIN");
    return e && *e ? (uint32_t)strtoul(e, nullptr, 10) : 4096u;
}
static bool sort_persist() {
    const char *e = getenv("XLOG_HIP_SORT_PERSIST");
    return e && e[0] == '1';
}

// The high-word route of a full-key sort (keys only, at least
// HYBRID_MIN_KEYS keys; XLOG_HIP_SORT_HYBRID=0 turns it off, read at each
// sort): when the high word splits the keys into runs of a few keys, the
// high word's digit passes and one short-run pass replace the low word's
// four digit passes.
constexpr uint64_t HYBRID_MIN_KEYS = 1ull << 22;
static bool sort_hybrid() {
    const char *e = getenv("XLOG_HIP_SORT_HYBRID");
    return !(e && e[0] == '0');
}
// From the digit histograms: is a key expected to share its high word with
// at most a few others?  sum_b h_d[b]^2 / n^2 is the chance that two keys
// drawn at random agree on digit d; the product over the high word's four
// digits, as if the digits were independent, estimates the chance that they
// agree on the whole high word.  Inputs where the estimate is wrong (digits
// that move together) have longer runs than predicted; a run of more than
// 256 keys is caught by the short-run pass, and the sort then runs every
// digit's pass.
static bool short_high_runs(const uint32_t *h, uint64_t n) {
    double p = 1.0;
    for (int d = 4; d < 8; ++d) {
        double s = 0.0;
        for (int b = 0; b < 256; ++b) s += (double)h[d * 256 + b] * (double)h[d * 256 + b];
        p *= s / ((double)n * (double)n);
    }
    return (double)(n - 1) * p <= 8.0;
}

// The segment route of a large full-key sort (keys only, at least
// XLOG_HIP_SORT_SEG_MIN keys, default 2^22), or of a sort of the high word
// whose caller accepts the whole key's order: two digit passes order the keys
// by their top 16 bits and one on-chip sort per segment (sort_top_segments)
// replaces the other digits' passes.  A segment is the keys of 2^gshift
// consecutive top-16-bit values, gshift the largest (at most 6) that keeps
// segments at 4,096 keys or fewer on average (0 at 2^28 keys, 4 at 2^24, 6
// at 2^22).  From the histograms of digits 6 and 7: the largest
// segment, as if the two digits were independent, is max h7 * (max over
// 2^gshift consecutive digit-6 values of their count) / n; the route is taken
// when that leaves room below the on-chip capacity (a segment above it is
// caught by the segment pass, and the sort then runs every digit's pass).
// XLOG_HIP_SORT_SEGMENTS=0 turns the route off and XLOG_HIP_SORT_SEG_GSHIFT
// fixes gshift (tests), both read at each sort.
static bool segment_route(const uint32_t *h, uint64_t n, int *gshift) {
    const char *off = getenv("XLOG_HIP_SORT_SEGMENTS");
    if (off && off[0] == '0') return false;
    const char *e = getenv("XLOG_HIP_SORT_SEG_MIN");
    const uint64_t min_keys = e && *e ? strtoull(e, nullptr, 10) : (1ull << 22);
    if (n < min_keys) return false;
    int g = 0;
    while (g < 6 && (n << (g + 1)) <= 4096ull * 65536ull) ++g;
    const char *fg = getenv("XLOG_HIP_SORT_SEG_GSHIFT");  // a fixed segment width (tests)
    if (fg && *fg) g = std::min(6, std::max(0, atoi(fg)));
    uint32_t m7 = 0;
    uint64_t m6 = 0;
    for (int b = 0; b < 256; ++b) m7 = std::max(m7, h[7 * 256 + b]);
    for (int j = 0; j < (256 >> g); ++j) {
        uint64_t c = 0;
        for (int b = j << g; b < ((j + 1) << g); ++b) c += h[6 * 256 + b];
        m6 = std::max(m6, c);
    }
    *gshift = g;
    return (double)m6 * (double)m7 / (double)n <= 0.85 * (double)SORT_SEGMENT_MAX;
}

void sort_short_runs(Ctx *ctx, const uint64_t *in, uint64_t n, uint64_t *out, uint64_t *d_long) {
    fill_u64(ctx, d_long, 0ull, 1);
    if (!n) return;
    const uint64_t blocks = (n + SR_CORE - 1) / SR_CORE;
    XH_REQUIRE(blocks < (1ull << 31), XLOG_HIP_CAPACITY_OVERFLOW, "short-run sort: input too large");
    Prof prof(ctx, XLOG_HIP_KERNEL_SORT_RUNS, 16.0 * (double)n);  // reads and writes every key once
    hipLaunchKernelGGL(k_sort_short_runs, dim3((unsigned)blocks), dim3(SR_BLOCK), 0, ctx->stream, in, n, out, d_long);
    XH_CHECK_HIP(hipGetLastError());
}

uint64_t *sort_grouped_dev(Ctx *ctx, uint64_t *keys, uint64_t *keys_alt, uint64_t n_bound, const uint64_t *d_n,
                           uint32_t known_digits, const uint32_t *stop, uint64_t *scratch) {
    if (n_bound == 0) return keys_alt;
    XH_REQUIRE(n_bound < (1ull << 30), XLOG_HIP_CAPACITY_OVERFLOW, "grouped sort: limited to 2^30 - 1 keys");
    uint64_t *d_long = scratch;
    uint32_t *skip = reinterpret_cast<uint32_t *>(scratch + 1);
    fill_u64(ctx, d_long, 0ull, 1);
    {
        Prof prof(ctx, XLOG_HIP_KERNEL_SORT_RUNS, 0.0);
        add_work_rows(ctx, prof.work(16.0), d_n, n_bound, 1, nullptr, 0, 0, nullptr, stop);  // every key read, written
        const uint64_t cores = (n_bound + SR_CORE - 1) / SR_CORE;
        hipLaunchKernelGGL(k_sort_short_runs_dev, dim3(persistent_grid(ctx, cores, 8)), dim3(SR_BLOCK), 0, ctx->stream,
                           keys, n_bound, d_n, keys_alt, d_long, stop);
        XH_CHECK_HIP(hipGetLastError());
    }
    // a run of more than SR_MAX keys: every digit pass, from the unsorted keys (their buffer is intact)
    hipLaunchKernelGGL(k_fallback_skip, dim3(1), dim3(1), 0, ctx->stream, d_long, stop, skip);
    XH_CHECK_HIP(hipGetLastError());
    uint64_t *a = keys, *b = keys_alt;
    radix_sort_dev(ctx, &a, &b, n_bound, d_n, known_digits, skip);
    if (a == keys)  // an even number of passes ends where the keys started: bring the result over
        hipLaunchKernelGGL(k_copy_dev, dim3(grid_for(n_bound, 256, (unsigned)ctx->num_cus * 8)), dim3(256), 0,
                           ctx->stream, keys, n_bound, d_n, keys_alt, skip);
    XH_CHECK_HIP(hipGetLastError());
    return keys_alt;
}

int radix_sort_dev(Ctx *ctx, uint64_t **keys, uint64_t **keys_alt, uint64_t n_bound, const uint64_t *d_n,
                   uint32_t known_digits, const uint32_t *stop) {
    XH_REQUIRE(known_digits, XLOG_HIP_INVALID_ARG, "radix sort with a device count: the digits must be known");
    XH_REQUIRE(n_bound < (1ull << 30), XLOG_HIP_CAPACITY_OVERFLOW,
               "radix sort: a single sort call is limited to 2^30 - 1 keys");
    if (n_bound == 0) return 0;
    const uint64_t tile_keys = (uint64_t)SORT_BLOCK_K * SORT_ITEMS_K;
    const uint64_t tiles = (n_bound + tile_keys - 1) / tile_keys;
    SortState &st = sort_state(ctx, tiles);
    uint32_t *hist = st.hist, *off = st.hist + 8 * 256;
    // persistent passes: at most the blocks the device holds, tickets from a counter zeroed per pass
    const uint32_t cap = pass_capacity<false, SORT_BLOCK_K, SORT_ITEMS_K>(ctx);
    const unsigned grid = (unsigned)std::min<uint64_t>(tiles, cap);
    unsigned long long *tk = ctx->tickets + PERSIST_TICKET_SLOT + 1;
    fill_u32(ctx, hist, 0u, 8 * 256);
    {
        Prof prof(ctx, XLOG_HIP_KERNEL_SORT_HIST, 0.0);
        add_work_rows(ctx, prof.work(8.0), d_n, n_bound, 1, nullptr, 0, 0, nullptr, stop);  // reads every key once
        const unsigned hg = grid_for(n_bound, (unsigned)(HIST_BLOCK * HIST_ITEMS) * 4, (unsigned)ctx->num_cus * 8);
        hipLaunchKernelGGL(k_hist8, dim3(hg), dim3(HIST_BLOCK), 0, ctx->stream, *keys, n_bound, hist, 0, 8, d_n,
                           stop);
        XH_CHECK_HIP(hipGetLastError());
        hipLaunchKernelGGL(k_digit_offsets, dim3(1), dim3(64), 0, ctx->stream, hist, off);
        XH_CHECK_HIP(hipGetLastError());
    }
    // The first pass reads a status buffer made clean over every tile; each pass clears the entries of
    // its tiles that hold keys in the next pass's buffer, which is all the next pass reads.  After the
    // sort neither buffer is known to be clean past those tiles: both are marked dirty over the bound.
    int cur = (st.dirty[0] == 0) ? 0 : (st.dirty[1] == 0 ? 1 : 0);
    if (st.dirty[cur]) {
        fill_u32(ctx, st.status[cur], 0u, st.dirty[cur] * 256);
        st.dirty[cur] = 0;
    }
    int passes = 0;
    for (int dgt = 0; dgt < 8; ++dgt) {
        if (!((known_digits >> dgt) & 1u)) continue;
        const int nxt = 1 - cur;
        Prof prof(ctx, XLOG_HIP_KERNEL_SORT_PASS, 0.0);
        add_work_rows(ctx, prof.work(16.0), d_n, n_bound, 1, nullptr, 0, 0, nullptr, stop);
        hipLaunchKernelGGL((k_onesweep<false, SORT_BLOCK_K, SORT_ITEMS_K>), dim3(grid), dim3(SORT_BLOCK_K), 0,
                           ctx->stream, *keys, *keys_alt, nullptr, nullptr, n_bound, (uint32_t)tiles, 8 * dgt,
                           off + dgt * 256, st.status[cur], st.status[nxt], 1u, tk, 0ull, d_n, stop, sort_spin_limit());
        XH_CHECK_HIP(hipGetLastError());
        std::swap(*keys, *keys_alt);
        cur = nxt;
        ++passes;
    }
    st.dirty[0] = std::max<uint64_t>(st.dirty[0], tiles);
    st.dirty[1] = std::max<uint64_t>(st.dirty[1], tiles);
    return passes;
}

int radix_sort_u64(Ctx *ctx, uint64_t **keys, uint64_t **keys_alt, uint32_t **vals, uint32_t **vals_alt,
                   uint64_t n, int digit_lo, int digit_hi, const uint64_t *src, uint32_t known_digits,
                   SortUnique *uq, bool *whole) {
    if (whole) *whole = false;
    if (n < 2 || digit_lo >= digit_hi) {
        if (src && n) XH_CHECK_HIP(hipMemcpyAsync(*keys, src, n * 8, hipMemcpyDeviceToDevice, ctx->stream));
        return 0;
    }
    XH_REQUIRE(!(src && vals && *vals), XLOG_HIP_INVALID_ARG, "radix sort: a separate source is keys-only");
    XH_REQUIRE(n < (1ull << 30), XLOG_HIP_CAPACITY_OVERFLOW,
               "radix sort: a single sort call is limited to 2^30 - 1 keys");
    const bool has_val = vals && *vals;
    const uint64_t tile_keys = has_val ? (uint64_t)SORT_BLOCK_V * SORT_ITEMS_V : (uint64_t)SORT_BLOCK_K * SORT_ITEMS_K;
    const uint64_t tiles = (n + tile_keys - 1) / tile_keys;
    SortState &st = sort_state(ctx, tiles);
    uint32_t *hist = st.hist, *off = st.hist + 8 * 256;
    const uint32_t cap = has_val ? pass_capacity<true, SORT_BLOCK_V, SORT_ITEMS_V>(ctx)
                                 : pass_capacity<false, SORT_BLOCK_K, SORT_ITEMS_K>(ctx);
    // chunks of 8 consecutive tiles (4 and 16 measured alike, 1 and 2 slower),
    // at most 1/16 of the blocks the device holds, and smaller when a sort
    // has few tiles so that it still spreads over the XCDs
    uint32_t chunk = cap / 16 < 8 ? (cap / 16 > 0 ? cap / 16 : 1) : 8;
    if (tiles / 64 < chunk) chunk = tiles / 64 > 0 ? (uint32_t)(tiles / 64) : 1;
    const uint64_t nchunks = (tiles + chunk - 1) / chunk;
    const unsigned grid = (unsigned)(8 * ((nchunks + 7) / 8) * chunk);  // blocks past the last tile exit

    // A large full-key sort may take the high-word route, whose decision and
    // passes need only the high word's histograms: they are counted first, and
    // the low word's only when a pass over a low digit is needed.
    // (a sort given known_digits takes exactly those passes, so it needs every digit's histogram)
    const bool hybrid_candidate =
        !has_val && !known_digits && digit_lo == 0 && digit_hi == 8 && n >= HYBRID_MIN_KEYS && sort_hybrid();
    // a sort of the high word that may order the keys by the whole key instead (the segment route)
    const bool word_candidate = whole && !has_val && !known_digits && digit_lo == 4 && digit_hi == 8 &&
                                n >= HYBRID_MIN_KEYS && sort_hybrid();
    auto histograms = [&](const uint64_t *from, int dlo, int dhi) {
        Prof prof(ctx, XLOG_HIP_KERNEL_SORT_HIST, 8.0 * (double)n);  // reads every key once
        // at least 4 rounds per block: every block ends with up to 2048 device-scope atomics, which cost more
        // than the counting when blocks have little to count (2^24 keys: 62 us with one round per block, 47 us
        // with 4, 60 us with 16)
        const unsigned hg = grid_for(n, (unsigned)(HIST_BLOCK * HIST_ITEMS) * 4, (unsigned)ctx->num_cus * 8);
        hipLaunchKernelGGL(k_hist8, dim3(hg), dim3(HIST_BLOCK), 0, ctx->stream, from, n, hist, dlo, dhi, nullptr,
                           nullptr);
        XH_CHECK_HIP(hipGetLastError());
        hipLaunchKernelGGL(k_digit_offsets, dim3(1), dim3(64), 0, ctx->stream, hist, off);
        XH_CHECK_HIP(hipGetLastError());
    };
    fill_u32(ctx, hist, 0u, 8 * 256);
    histograms(src ? src : *keys, hybrid_candidate ? 4 : digit_lo, digit_hi);
    int passes = 0;
    int cur = 0;  // status buffer for the next pass
    if (st.dirty[0] == 0) cur = 0; else if (st.dirty[1] == 0) cur = 1; else cur = 0;
    auto launch_pass = [&](int dgt) {
        int nxt = 1 - cur;
        if (st.dirty[cur]) {  // make the buffer this pass reads clean
            fill_u32(ctx, st.status[cur], 0u, st.dirty[cur] * 256);
            st.dirty[cur] = 0;
        }
        Prof prof(ctx, XLOG_HIP_KERNEL_SORT_PASS, (has_val ? 24.0 : 16.0) * (double)n);
        unsigned long long *tk = pass_tickets() ? ctx->tickets + 2 : nullptr;
        unsigned long long tb = tk ? ctx->take_tickets(2, grid) : 0ull;
        // tickets go to tiles in plain order (chunk 1: chunk_tile is then the identity), which measured
        // faster than tickets dealt to XCD chunks
        const uint32_t pchunk = tk ? 1u : chunk;
        unsigned pgrid = grid;
        const uint64_t *pn = nullptr;
        if (sort_persist()) {
            // persistent: at most the blocks the device holds, tickets in plain order from the self-resetting
            // counter, the key count from a device word (every tile holds keys, so each pass clears all of
            // the next pass's `tiles` entries, as the index-ordered pass does)
            tk = ctx->tickets + PERSIST_TICKET_SLOT + 1;
            tb = 0;
            pn = reinterpret_cast<const uint64_t *>(ctx->tickets + 12);
            fill_u64(ctx, reinterpret_cast<uint64_t *>(ctx->tickets + 12), n, 1);
            pgrid = (unsigned)std::min<uint64_t>(tiles, cap);
        }
        if (has_val)
            hipLaunchKernelGGL((k_onesweep<true, SORT_BLOCK_V, SORT_ITEMS_V>), dim3(pgrid), dim3(SORT_BLOCK_V), 0,
                               ctx->stream, *keys, *keys_alt, *vals, *vals_alt, n, (uint32_t)tiles, 8 * dgt,
                               off + dgt * 256, st.status[cur], st.status[nxt], pchunk, tk, tb, pn, nullptr,
                               sort_spin_limit());
        else
            hipLaunchKernelGGL((k_onesweep<false, SORT_BLOCK_K, SORT_ITEMS_K>), dim3(pgrid), dim3(SORT_BLOCK_K), 0,
                               ctx->stream, (passes == 0 && src) ? src : *keys, *keys_alt, nullptr, nullptr, n,
                               (uint32_t)tiles, 8 * dgt, off + dgt * 256, st.status[cur], st.status[nxt], pchunk,
                               tk, tb, pn, nullptr, sort_spin_limit());
        XH_CHECK_HIP(hipGetLastError());
        st.dirty[cur] = tiles;
        if (st.dirty[nxt] <= tiles) st.dirty[nxt] = 0;
        std::swap(*keys, *keys_alt);
        if (has_val) std::swap(*vals, *vals_alt);
        cur = nxt;
        ++passes;
    };
    if (known_digits) {  // the caller knows which digits may vary: no read-back
        for (int dgt = digit_lo; dgt < digit_hi; ++dgt)
            if ((known_digits >> dgt) & 1u) launch_pass(dgt);
        if (passes == 0 && src) XH_CHECK_HIP(hipMemcpyAsync(*keys, src, n * 8, hipMemcpyDeviceToDevice, ctx->stream));
        return passes;
    }
    // The host copy of the histograms decides which digit passes are needed.
    // The pass of the lowest digit is launched before waiting for it (a pass
    // over a constant digit is a stable copy, so it is right either way): the
    // device works on it while the host reads the histograms and queues the
    // rest, instead of idling through the read-back.  A large full-key sort
    // waits instead, since its histograms may choose the high-word route.
    uint32_t h_hist[8 * 256];
    static_assert(sizeof(h_hist) <= Ctx::HOST_STAGE_U64 * sizeof(uint64_t), "histograms exceed the staging");
    XH_CHECK_HIP(hipMemcpyAsync(ctx->host_scalars, hist, sizeof(h_hist), hipMemcpyDeviceToHost, ctx->stream));
    XH_CHECK_HIP(hipEventRecord(ctx->ev_read, ctx->stream));
    int first = digit_lo;
    if (digit_hi - digit_lo >= 2 && !hybrid_candidate && !word_candidate) launch_pass(first++);
    ctx->wait_event(ctx->ev_read);
    memcpy(h_hist, ctx->host_scalars, sizeof(h_hist));
    auto trivial = [&](int dgt) {
        for (int b = 0; b < 256; ++b)
            if (h_hist[dgt * 256 + b] == n) return true;
        return false;
    };
    // the low word's histograms (their counters are still zero) from the same multiset of keys, and back
    auto low_word_histograms = [&](const uint64_t *from) {
        histograms(from, 0, 4);
        XH_CHECK_HIP(hipMemcpyAsync(ctx->host_scalars, hist, sizeof(h_hist), hipMemcpyDeviceToHost, ctx->stream));
        XH_CHECK_HIP(hipEventRecord(ctx->ev_read, ctx->stream));
        ctx->wait_event(ctx->ev_read);
        memcpy(h_hist, ctx->host_scalars, sizeof(h_hist));
    };
    int gshift = 0;
    if ((hybrid_candidate || word_candidate) && segment_route(h_hist, n, &gshift)) {
        // The top two digits, then every segment sorted on chip.
        for (int dgt = 6; dgt < 8; ++dgt)
            if (!trivial(dgt)) launch_pass(dgt);
        Buf<uint64_t> flags(ctx, 2);  // unique count (with uq), long segment or run
        sort_top_segments(ctx, (passes == 0 && src) ? src : *keys, n, *keys_alt, uq ? flags.p : nullptr,
                          flags.p + 1, gshift);
        ctx->read_scalars(flags.p, 2);
        if (ctx->host_scalars[1] == 0) {
            if (uq) {
                uq->done = true;
                uq->count = ctx->host_scalars[0];
            }
            std::swap(*keys, *keys_alt);
            if (whole) *whole = true;
            return passes + 1;
        }
        // a segment above the on-chip capacity or a long run of unequal keys:
        // every digit's pass of the sort, from the keys as they are (any order
        // sorts alike)
        if (word_candidate) {
            for (int dgt = 4; dgt < 8; ++dgt)
                if (!trivial(dgt)) launch_pass(dgt);
            return passes;
        }
        low_word_histograms((passes == 0 && src) ? src : *keys);
        for (int dgt = 0; dgt < 8; ++dgt)
            if (!trivial(dgt)) launch_pass(dgt);
        return passes;
    }
    if (hybrid_candidate && short_high_runs(h_hist, n)) {
        // The high word's passes, then every run of equal high word sorted by
        // its low word in one pass instead of the low word's four passes.
        for (int dgt = 4; dgt < 8; ++dgt)
            if (!trivial(dgt)) launch_pass(dgt);
        if (passes > 0) {
            Buf<uint64_t> flags(ctx, 2);  // unique count (with uq), long run
            if (uq) sort_short_runs_unique(ctx, *keys, n, *keys_alt, flags.p, flags.p + 1);
            else sort_short_runs(ctx, *keys, n, *keys_alt, flags.p + 1);
            ctx->read_scalars(flags.p, 2);
            if (ctx->host_scalars[1] == 0) {
                if (uq) {
                    uq->done = true;
                    uq->count = ctx->host_scalars[0];
                }
                std::swap(*keys, *keys_alt);
                return passes + 1;
            }
            // a run of more than 256 keys: *keys (the keys sorted by their
            // high word, intact) takes every digit's pass; any order of the
            // keys sorts to the same result
            low_word_histograms(*keys);
            for (int dgt = 0; dgt < 8; ++dgt)
                if (!trivial(dgt)) launch_pass(dgt);
            return passes;
        }
    }
    if (hybrid_candidate) low_word_histograms(src ? src : *keys);
    for (int dgt = first; dgt < digit_hi; ++dgt)
        if (!trivial(dgt)) launch_pass(dgt);
    if (passes == 0 && src) XH_CHECK_HIP(hipMemcpyAsync(*keys, src, n * 8, hipMemcpyDeviceToDevice, ctx->stream));
    return passes;
}

}  // namespace xh
