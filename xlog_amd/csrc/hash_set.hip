// Device hash set of packed u64 tuples for gfx950, and the sparse factorized
// delta step built on it.
//
// Replaces the reference's sparse-domain factorized delta
// (fj_delta_sparse_novel_u32_recorded, crates/xlog-cuda/src/provider/fj_delta_sparse.rs:66;
// kernels wcoj.cu:4008-4121), which rebuilds an open-addressing set from the
// full relation for every step and scans its slots for the novel tuples.
// Here the set persists across the iterations of a fixpoint: it IS the full
// relation R, so one fused pass per iteration
//   - expands every delta row (carry, key) through the edge relation's run
//     index (the join build of join.hip: 16-byte slots key -> run),
//   - inserts (carry, value) with a 64-bit compare-and-swap, and
//   - appends the tuples it inserted (the novel ones) to the next delta,
// so `(delta join edge) \ R`, the merge R |= delta' and the dedup of the
// candidates are one pass with no sort, and the host reads back one count
// per iteration.  R is sorted once, at the end.
//
// Slots hold the key itself; the empty slot is all ones.  The key
// (0xFFFFFFFF, 0xFFFFFFFF) cannot be stored in a slot, so its presence is a
// separate flag.  Linear probing, Fibonacci hashing of the whole key.
#include "internal.hpp"

#include <algorithm>

namespace xh {

namespace {

constexpr uint64_t HS_EMPTY = ~0ull;
constexpr int HB = 256;  // block of the insert kernels

struct SetView {
    unsigned long long *slots;
    uint64_t mask;
    int bits;
    unsigned int *allones;  // 1 when the all-ones key is present
};

__device__ __forceinline__ uint64_t hs_hash(uint64_t k, int bits) {
    k ^= k >> 31;
    return (uint64_t)((k * 0x9E3779B97F4A7C15ull) >> (64 - bits));
}

// 1: inserted (the key was absent), 0: present already, 2: the table is full.
// A slot changes once, from empty to its key, so a plain (cacheable) load is
// enough: a stale "empty" only sends the lane to the compare-and-swap, which
// returns the slot's real value.
__device__ __forceinline__ int hs_insert(const SetView &s, uint64_t key) {
    if (key == HS_EMPTY) return atomicExch(s.allones, 1u) == 0u ? 1 : 0;
    uint64_t h = hs_hash(key, s.bits);
    for (uint64_t p = 0; p <= s.mask; ++p) {
        const unsigned long long cur = s.slots[h];
        if (cur == key) return 0;
        if (cur == HS_EMPTY) {
            const unsigned long long prev = atomicCAS(&s.slots[h], HS_EMPTY, (unsigned long long)key);
            if (prev == HS_EMPTY) return 1;
            if (prev == key) return 0;
        }
        h = (h + 1) & s.mask;
    }
    return 2;
}

// hs_insert with the first slot already loaded (cur = slots[h], h = the key's
// home slot): callers issue the first loads of several keys together.
__device__ __forceinline__ int hs_insert_from(const SetView &s, uint64_t key, uint64_t h, unsigned long long cur) {
    if (key == HS_EMPTY) return atomicExch(s.allones, 1u) == 0u ? 1 : 0;
    for (uint64_t p = 0; p <= s.mask; ++p) {
        if (p) cur = s.slots[h];
        if (cur == key) return 0;
        if (cur == HS_EMPTY) {
            const unsigned long long prev = atomicCAS(&s.slots[h], HS_EMPTY, (unsigned long long)key);
            if (prev == HS_EMPTY) return 1;
            if (prev == key) return 0;
        }
        h = (h + 1) & s.mask;
    }
    return 2;
}

// Keys handled per lane per chunk by the insert kernels: their first probes are
// in flight together.
constexpr int HS_U = 4;

// Appends up to HS_U novel keys per lane with one atomic per wave (a wave scan
// of the per-lane counts) and returns the count after it (0 when nothing was
// appended).
__device__ __forceinline__ uint64_t wave_append_n(const bool *novel, const uint64_t *key, uint64_t *out,
                                                  unsigned long long *count, int lane) {
    uint32_t c = 0;
#pragma unroll
    for (int u = 0; u < HS_U; ++u) c += novel[u] ? 1u : 0u;
    uint32_t incl = c;
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
        const uint32_t t = __shfl_up(incl, o, WAVE);
        if (lane >= o) incl += t;
    }
    const uint32_t tot = __shfl(incl, WAVE - 1, WAVE);
    if (tot == 0) return 0;
    unsigned long long base = 0;
    if (lane == WAVE - 1) base = atomicAdd(count, (unsigned long long)tot);
    base = __shfl(base, WAVE - 1, WAVE);
    uint64_t pos = base + (incl - c);
#pragma unroll
    for (int u = 0; u < HS_U; ++u)
        if (novel[u]) out[pos++] = key[u];
    return base + tot;
}

// Appends the lanes' novel keys of one round with one atomic per wave and
// returns the count after it (0 when nothing was appended).  The caller's
// overflow protocol (k_hs_join_insert) keeps the count within the output's
// capacity.
__device__ __forceinline__ uint64_t wave_append(bool novel, uint64_t key, uint64_t *out, unsigned long long *count,
                                                int lane) {
    const uint64_t m = __ballot(novel);
    if (!m) return 0;
    unsigned long long base = 0;
    const int leader = __builtin_ctzll(m);
    const unsigned long long add = (unsigned long long)__popcll(m);
    if (lane == leader) base = atomicAdd(count, add);
    base = __shfl(base, leader, WAVE);
    if (novel) out[base + (uint64_t)__popcll(m & ((1ull << lane) - 1ull))] = key;
    return base + add;
}
// a full table seen by any lane stops the wave
__device__ __forceinline__ bool any_full(bool full) { return __ballot(full) != 0ull; }

// A queued step's row count and limit (QueuedStep); false when an earlier
// step overflowed and this one is to do nothing.  Every thread reads the
// same words, written by earlier launches, so the answer is uniform.
__device__ __forceinline__ bool queued_prologue(const QueuedStep &q, uint64_t &n, uint64_t &limit) {
    uint64_t used = 0;
    for (int t = 0; t < q.nprior; ++t) {
        if (q.stop[t]) return false;
        used += q.prior[(uint64_t)t * q.stride];
    }
    if (q.d_n && *q.d_n < n) n = *q.d_n;
    const uint64_t left = used < q.room ? q.room - used : 0;
    if (left < limit) limit = left;
    return true;
}

// Inserts keys[0..n) (no novelty bookkeeping): the initial full relation
// (rehash = 0: the all-ones key is a tuple and sets its flag), or the slots
// of an old table being rehashed (rehash = 1: all ones is an empty slot and is
// skipped; the flag carries over with the table's flags).
__global__ void k_hs_insert_all(const uint64_t *__restrict__ keys, uint64_t n, SetView s,
                                unsigned long long *overflow, int rehash) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i0 = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i0 < n; i0 += stride * HS_U) {
        uint64_t k[HS_U], h[HS_U];
        unsigned long long cur[HS_U];
#pragma unroll
        for (int u = 0; u < HS_U; ++u) {
            const uint64_t i = i0 + (uint64_t)u * stride;
            k[u] = i < n ? keys[i] : HS_EMPTY;  // past the end: nothing to insert
            if (i < n && k[u] == HS_EMPTY && !rehash) atomicExch(s.allones, 1u);
        }
#pragma unroll
        for (int u = 0; u < HS_U; ++u) {
            h[u] = hs_hash(k[u], s.bits);
            cur[u] = k[u] != HS_EMPTY ? s.slots[h[u]] : 0ull;
        }
#pragma unroll
        for (int u = 0; u < HS_U; ++u)
            if (k[u] != HS_EMPTY && hs_insert_from(s, k[u], h[u], cur[u]) == 2) *overflow = 1ull;
    }
}

// Inserts keys[0..n) and appends the novel ones to out (capacity limit):
// the generic set-difference-and-merge of a candidate bag.
// With swap the keys' words are exchanged first; q is a queued step or
// empty.
__global__ __launch_bounds__(HB) void k_hs_insert_novel(const uint64_t *__restrict__ keys, uint64_t n, SetView s,
                                                        uint64_t *__restrict__ out, unsigned long long *count,
                                                        uint64_t limit, unsigned long long *overflow, int swap,
                                                        QueuedStep q, unsigned long long *work) {
    if (!queued_prologue(q, n, limit)) return;
    if (work && blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(work, 16ull * n);  // algorithmic: key + slot
    const int lane = threadIdx.x & (WAVE - 1);
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    // whole waves step together so that the append's ballot sees every lane
    for (uint64_t base = (uint64_t)blockIdx.x * blockDim.x + (threadIdx.x & ~(WAVE - 1)); base < n; base += stride) {
        const uint64_t i = base + lane;
        bool novel = false, full = false;
        uint64_t k = 0;
        if (i < n) {
            k = keys[i];
            if (swap) k = (k << 32) | (k >> 32);
            const int r = hs_insert(s, k);
            full = r == 2;
            novel = r == 1;
        }
        const uint64_t after = wave_append(novel, k, out, count, lane);
        if (after >= limit || any_full(full)) {
            if (lane == 0) *overflow = 1ull;
            return;
        }
    }
}

// Run index lookup (the 16-byte slots of join.hip's build: (key << 32) | run
// length, run start; a run is never empty, so 0 marks an empty slot).
typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint64_t run_hash(uint32_t key, int bits) {
    return (uint64_t)(((uint64_t)key * 0x9E3779B97F4A7C15ull) >> (64 - bits));
}
__device__ __forceinline__ void run_lookup(const unsigned long long *table, uint64_t mask, int bits, uint32_t key,
                                           uint64_t *start, uint32_t *len) {
    uint64_t h = run_hash(key, bits);
    for (;;) {
        const u64x2 sl = *reinterpret_cast<const u64x2 *>(table + 2 * h);
        if (sl.x == 0ull) {
            *start = 0;
            *len = 0;
            return;
        }
        if ((uint32_t)(sl.x >> 32) == key) {
            *start = sl.y;
            *len = (uint32_t)sl.x;
            return;
        }
        h = (h + 1) & mask;
    }
}

struct JoinInsertArgs {
    const uint64_t *delta;  // packed delta rows
    uint64_t n;
    int key_hi;             // the join key is the high word of a delta row (else the low word)
    int out_carry_hi;       // the carried column goes to the high word of the head (else the low word)
    const unsigned long long *table;  // run index over the edge relation's join column
    uint64_t table_mask;
    int table_bits;
    const uint32_t *payload;          // edge value column, run order
};

// One sparse factorized delta step: for every delta row (carry, key) and every
// edge (key, value), insert head(carry, value); append the inserted ones.
// A wave takes 64 delta rows per round, looks their runs up, scans the run
// lengths and expands them 64 outputs at a time (lane j takes outputs j, j+64,
// ... of the round; its row is found by a 6-step search over the wave's
// prefixes in LDS), so a hub's long run is shared by the whole wave.
// Overflow protocol: a wave whose append returns a count at or past `limit`,
// or that finds the table full, raises the overflow flag and stops.  The
// append's atomic returns the count to every appending wave, so after the
// count passes `limit` each wave of the grid appends at most one more chunk
// (64 x HS_U tuples: its next append sees the count), which the output's slack
// (HS_APPEND_SLACK >= 64 x HS_U x the grid's waves) covers; no wave polls a
// shared word.  The host then grows the table / output and runs the step
// again: tuples inserted by the first run are found present and not appended
// twice, so the appended list is exactly the novel set.
__global__ __launch_bounds__(HB) void k_hs_join_insert(JoinInsertArgs a, SetView s, uint64_t *__restrict__ out,
                                                       unsigned long long *count, uint64_t limit,
                                                       unsigned long long *overflow,
                                                       unsigned long long *work) {
    __shared__ uint64_t s_pre[HB / WAVE][WAVE];  // exclusive prefix of run lengths per wave round
    __shared__ uint64_t s_start[HB / WAVE][WAVE];
    __shared__ uint32_t s_carry[HB / WAVE][WAVE];
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const uint64_t gwave = (uint64_t)blockIdx.x * (HB / WAVE) + (uint64_t)wave;
    const uint64_t nwaves = (uint64_t)gridDim.x * (HB / WAVE);
    unsigned long long cand = 0;
    for (uint64_t rbase = gwave * WAVE; rbase < a.n; rbase += nwaves * WAVE) {
        const uint64_t i = rbase + lane;
        uint64_t st = 0;
        uint32_t len = 0, carry = 0;
        if (i < a.n) {
            const uint64_t row = a.delta[i];
            const uint32_t key = a.key_hi ? (uint32_t)(row >> 32) : (uint32_t)row;
            carry = a.key_hi ? (uint32_t)row : (uint32_t)(row >> 32);
            run_lookup(a.table, a.table_mask, a.table_bits, key, &st, &len);
        }
        // wave exclusive scan of the run lengths
        uint64_t incl = len;
#pragma unroll
        for (int o = 1; o < WAVE; o <<= 1) {
            const uint64_t t = __shfl_up(incl, o, WAVE);
            if (lane >= o) incl += t;
        }
        const uint64_t total = __shfl(incl, WAVE - 1, WAVE);
        s_pre[wave][lane] = incl - len;
        s_start[wave][lane] = st;
        s_carry[wave][lane] = carry;
        __builtin_amdgcn_wave_barrier();
        cand += total;
        for (uint64_t ob = 0; ob < total; ob += (uint64_t)WAVE * HS_U) {
            // HS_U outputs per lane: their payload loads, then their first slot loads, are in flight together
            uint64_t key[HS_U], h[HS_U];
            unsigned long long cur[HS_U];
            bool valid[HS_U], novel[HS_U], full = false;
#pragma unroll
            for (int u = 0; u < HS_U; ++u) {
                const uint64_t o = ob + (uint64_t)u * WAVE + lane;
                valid[u] = o < total;
                // last row r with s_pre[r] <= o (rows with empty runs share their prefix with the next row,
                // so the search lands on a row with a non-empty run)
                int r = 0;
#pragma unroll
                for (int step = 32; step > 0; step >>= 1)
                    if (s_pre[wave][r + step] <= o) r += step;
                const uint32_t z = valid[u] ? a.payload[s_start[wave][r] + (o - s_pre[wave][r])] : 0u;
                const uint32_t x = s_carry[wave][r];
                key[u] = a.out_carry_hi ? (((uint64_t)x << 32) | z) : (((uint64_t)z << 32) | x);
            }
#pragma unroll
            for (int u = 0; u < HS_U; ++u) {
                h[u] = hs_hash(key[u], s.bits);
                cur[u] = (valid[u] && key[u] != HS_EMPTY) ? s.slots[h[u]] : 0ull;
            }
#pragma unroll
            for (int u = 0; u < HS_U; ++u) {
                const int res = valid[u] ? hs_insert_from(s, key[u], h[u], cur[u]) : 0;
                full |= res == 2;
                novel[u] = res == 1;
            }
            const uint64_t after = wave_append_n(novel, key, out, count, lane);
            if (after >= limit || any_full(full)) {
                if (lane == 0) *overflow = 1ull;
                return;
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
    if (work) {
        // algorithmic bytes: delta row + run slot per row, value + slot per candidate (added per wave)
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) cand += __shfl_xor(cand, o, WAVE);
        if (lane == 0) atomicAdd(work + (blockIdx.x & 63), cand * 12ull);
    }
}

// One step of a path-shaped rule body over the hash set of its head, for
// bodies of up to three atoms (two hops besides the delta atom): every delta
// row (xa, xb) (the delta atom's two path values) is expanded through hop 1
// (a run of values v1 for xa or xb) and, when the body has a third atom,
// each level-1 value through hop 2 (a run of values v2 for xa, xb or v1), and
// the head tuple built from (xa, xb, v1, v2) is inserted; the inserted ones
// are appended.  Nothing between the levels leaves the wave: level-1 values
// are expanded 64 at a time (one per lane, found by a search over the wave's
// run-length prefixes in LDS) and their level-2 runs 64 x HS_U outputs at a
// time, so the binary intermediate of the first two atoms is never written.
// The overflow protocol is that of k_hs_join_insert.
__device__ __forceinline__ uint32_t path_val(int sel, uint32_t xa, uint32_t xb, uint32_t v1, uint32_t v2) {
    return sel == 0 ? xa : sel == 1 ? xb : sel == 2 ? v1 : v2;
}
__device__ __forceinline__ int last_le(const uint64_t *pre, uint64_t o) {
    int r = 0;
#pragma unroll
    for (int step = 32; step > 0; step >>= 1)
        if (pre[r + step] <= o) r += step;
    return r;
}

template <bool TWO>
__global__ __launch_bounds__(HB) void k_hs_path_insert(PathInsertArgs a, SetView s, uint64_t *__restrict__ out,
                                                       unsigned long long *count, uint64_t limit,
                                                       unsigned long long *overflow, unsigned long long *work) {
    __shared__ uint64_t s_pre1[HB / WAVE][WAVE], s_st1[HB / WAVE][WAVE];
    __shared__ uint32_t s_xa[HB / WAVE][WAVE], s_xb[HB / WAVE][WAVE];
    __shared__ uint64_t s_pre2[TWO ? HB / WAVE : 1][WAVE], s_st2[TWO ? HB / WAVE : 1][WAVE];
    __shared__ uint32_t s_v1[TWO ? HB / WAVE : 1][WAVE], s_ra[TWO ? HB / WAVE : 1][WAVE],
        s_rb[TWO ? HB / WAVE : 1][WAVE];
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const uint64_t gwave = (uint64_t)blockIdx.x * (HB / WAVE) + (uint64_t)wave;
    const uint64_t nwaves = (uint64_t)gridDim.x * (HB / WAVE);
    uint64_t n = a.n;
    if (!queued_prologue(a.q, n, limit)) return;  // an earlier queued step overflowed
    if (work && blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(work, 24ull * n);
    unsigned long long cand = 0;
    for (uint64_t rbase = gwave * WAVE; rbase < n; rbase += nwaves * WAVE) {
        const uint64_t i = rbase + lane;
        uint32_t xa = 0, xb = 0, len1 = 0;
        uint64_t st1 = 0;
        if (i < n) {
            const uint64_t row = a.delta[i];
            xa = a.delta_swap ? (uint32_t)row : (uint32_t)(row >> 32);
            xb = a.delta_swap ? (uint32_t)(row >> 32) : (uint32_t)row;
            run_lookup(a.h1.table, a.h1.mask, a.h1.bits, a.key1 ? xb : xa, &st1, &len1);
        }
        uint64_t incl = len1;
#pragma unroll
        for (int o = 1; o < WAVE; o <<= 1) {
            const uint64_t t = __shfl_up(incl, o, WAVE);
            if (lane >= o) incl += t;
        }
        const uint64_t total1 = __shfl(incl, WAVE - 1, WAVE);
        s_pre1[wave][lane] = incl - len1;
        s_st1[wave][lane] = st1;
        s_xa[wave][lane] = xa;
        s_xb[wave][lane] = xb;
        __builtin_amdgcn_wave_barrier();
        if constexpr (!TWO) {
            cand += total1;
            for (uint64_t ob = 0; ob < total1; ob += (uint64_t)WAVE * HS_U) {
                uint64_t key[HS_U], h[HS_U];
                unsigned long long cur[HS_U];
                bool valid[HS_U], novel[HS_U], full = false;
#pragma unroll
                for (int u = 0; u < HS_U; ++u) {
                    const uint64_t o = ob + (uint64_t)u * WAVE + lane;
                    valid[u] = o < total1;
                    const int r = last_le(s_pre1[wave], o);
                    const uint32_t v1 = valid[u] ? a.h1.payload[s_st1[wave][r] + (o - s_pre1[wave][r])] : 0u;
                    const uint32_t ra = s_xa[wave][r], rb = s_xb[wave][r];
                    key[u] = ((uint64_t)path_val(a.out0, ra, rb, v1, 0u) << 32) | path_val(a.out1, ra, rb, v1, 0u);
                }
#pragma unroll
                for (int u = 0; u < HS_U; ++u) {
                    h[u] = hs_hash(key[u], s.bits);
                    cur[u] = (valid[u] && key[u] != HS_EMPTY) ? s.slots[h[u]] : 0ull;
                }
#pragma unroll
                for (int u = 0; u < HS_U; ++u) {
                    const int res = valid[u] ? hs_insert_from(s, key[u], h[u], cur[u]) : 0;
                    full |= res == 2;
                    novel[u] = res == 1;
                }
                const uint64_t after = wave_append_n(novel, key, out, count, lane);
                if (after >= limit || any_full(full)) {
                    if (lane == 0) *overflow = 1ull;
                    return;
                }
            }
        } else {
            for (uint64_t o1b = 0; o1b < total1; o1b += WAVE) {
                // one level-1 value per lane, then its hop-2 run
                const uint64_t o1 = o1b + lane;
                const bool valid1 = o1 < total1;
                const int r = last_le(s_pre1[wave], valid1 ? o1 : 0);
                const uint32_t ra = s_xa[wave][r], rb = s_xb[wave][r];
                const uint32_t v1 = valid1 ? a.h1.payload[s_st1[wave][r] + (o1 - s_pre1[wave][r])] : 0u;
                uint64_t st2 = 0;
                uint32_t len2 = 0;
                if (valid1) run_lookup(a.h2.table, a.h2.mask, a.h2.bits, path_val(a.key2, ra, rb, v1, 0u), &st2, &len2);
                uint64_t incl2 = len2;
#pragma unroll
                for (int o = 1; o < WAVE; o <<= 1) {
                    const uint64_t t = __shfl_up(incl2, o, WAVE);
                    if (lane >= o) incl2 += t;
                }
                const uint64_t total2 = __shfl(incl2, WAVE - 1, WAVE);
                __builtin_amdgcn_wave_barrier();  // the previous round's readers are done
                s_pre2[wave][lane] = incl2 - len2;
                s_st2[wave][lane] = st2;
                s_v1[wave][lane] = v1;
                s_ra[wave][lane] = ra;
                s_rb[wave][lane] = rb;
                __builtin_amdgcn_wave_barrier();
                cand += total2;
                for (uint64_t ob = 0; ob < total2; ob += (uint64_t)WAVE * HS_U) {
                    uint64_t key[HS_U], h[HS_U];
                    unsigned long long cur[HS_U];
                    bool valid[HS_U], novel[HS_U], full = false;
#pragma unroll
                    for (int u = 0; u < HS_U; ++u) {
                        const uint64_t o = ob + (uint64_t)u * WAVE + lane;
                        valid[u] = o < total2;
                        const int q = last_le(s_pre2[wave], o);
                        const uint32_t v2 = valid[u] ? a.h2.payload[s_st2[wave][q] + (o - s_pre2[wave][q])] : 0u;
                        const uint32_t qa = s_ra[wave][q], qb = s_rb[wave][q], qv = s_v1[wave][q];
                        key[u] = ((uint64_t)path_val(a.out0, qa, qb, qv, v2) << 32) | path_val(a.out1, qa, qb, qv, v2);
                    }
#pragma unroll
                    for (int u = 0; u < HS_U; ++u) {
                        h[u] = hs_hash(key[u], s.bits);
                        cur[u] = (valid[u] && key[u] != HS_EMPTY) ? s.slots[h[u]] : 0ull;
                    }
#pragma unroll
                    for (int u = 0; u < HS_U; ++u) {
                        const int res = valid[u] ? hs_insert_from(s, key[u], h[u], cur[u]) : 0;
                        full |= res == 2;
                        novel[u] = res == 1;
                    }
                    const uint64_t after = wave_append_n(novel, key, out, count, lane);
                    if (after >= limit || any_full(full)) {
                        if (lane == 0) *overflow = 1ull;
                        return;
                    }
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
    if (work) {
        // algorithmic bytes: per candidate its value (4 B) + slot word (8 B); the delta row + run slot per
        // row (24 B) are added above
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) cand += __shfl_xor(cand, o, WAVE);
        if (lane == 0) atomicAdd(work + (blockIdx.x & 63), cand * 12ull);
    }
}

__global__ void k_hs_append_allones(const unsigned int *allones, uint64_t *out, uint64_t *count) {
    if (*allones) out[(*count)++] = HS_EMPTY;
}

}  // namespace

// ---- host side --------------------------------------------------------------

static SetView view(const HashSet &h) {
    return SetView{reinterpret_cast<unsigned long long *>(h.slots.p), h.cap - 1, h.bits,
                   reinterpret_cast<unsigned int *>(h.flags.p)};
}

void hs_init(Ctx *ctx, HashSet &h, uint64_t min_cap) {
    int bits = 6;
    while ((1ull << bits) < min_cap) ++bits;
    XH_REQUIRE(bits <= 40, XLOG_HIP_CAPACITY_OVERFLOW, "hash set: more than 2^40 slots");
    h.bits = bits;
    h.cap = 1ull << bits;
    h.slots = Buf<uint64_t>(ctx, h.cap);
    fill_u64(ctx, h.slots.p, HS_EMPTY, h.cap);
    // flags: [0] all-ones key present (u32), [1] overflow, [2] appended count
    if (!h.flags.p) h.flags = Buf<uint64_t>(ctx, 4);
    fill_u64(ctx, h.flags.p, 0ull, 4);
    h.size = 0;
}

// Grids of the novel-insert kernels: at most HS_APPEND_SLACK / 64 waves, so
// that the appends past the limit (one chunk per wave) fit the slack.
constexpr unsigned HS_MAX_BLOCKS = (unsigned)(HS_APPEND_SLACK / ((uint64_t)WAVE * HS_U) / (HB / WAVE));
static unsigned grid_blocks(Ctx *ctx, uint64_t threads) {
    return grid_for(threads, HB, std::min<unsigned>((unsigned)ctx->num_cus * 16, HS_MAX_BLOCKS));
}

static void insert_all(Ctx *ctx, HashSet &h, const uint64_t *keys, uint64_t n, int rehash) {
    if (!n) return;
    unsigned long long *ovf = reinterpret_cast<unsigned long long *>(h.flags.p + 1);
    hipLaunchKernelGGL(k_hs_insert_all, dim3(grid_blocks(ctx, n)), dim3(HB), 0, ctx->stream, keys, n, view(h), ovf,
                       rehash);
    XH_CHECK_HIP(hipGetLastError());
}
void hs_insert_all(Ctx *ctx, HashSet &h, const uint64_t *keys, uint64_t n) { insert_all(ctx, h, keys, n, 0); }

void hs_grow(Ctx *ctx, HashSet &h, uint64_t min_cap) {
    HashSet g;
    g.flags = std::move(h.flags);  // the all-ones flag carries over; overflow is cleared below
    int bits = h.bits;
    while ((1ull << bits) < min_cap) ++bits;
    XH_REQUIRE(bits <= 40, XLOG_HIP_CAPACITY_OVERFLOW, "hash set: more than 2^40 slots");
    g.bits = bits;
    g.cap = 1ull << bits;
    g.slots = Buf<uint64_t>(ctx, g.cap);
    fill_u64(ctx, g.slots.p, HS_EMPTY, g.cap);
    fill_u64(ctx, g.flags.p + 1, 0ull, 1);
    insert_all(ctx, g, h.slots.p, h.cap, 1);  // skips the empty slots
    g.size = h.size;
    h = std::move(g);
}

void hs_join_insert(Ctx *ctx, HashSet &h, const uint64_t *delta, uint64_t n, int key_hi, int out_carry_hi,
                    const RunIndex &ix, const uint32_t *payload, uint64_t *out, uint64_t limit) {
    if (!n) return;
    JoinInsertArgs a;
    a.delta = delta;
    a.n = n;
    a.key_hi = key_hi;
    a.out_carry_hi = out_carry_hi;
    a.table = ix.table.p;
    a.table_mask = ix.table_mask;
    int tb = 0;
    while ((1ull << tb) < ix.table_mask + 1) ++tb;
    a.table_bits = tb;
    a.payload = payload;
    unsigned long long *ovf = reinterpret_cast<unsigned long long *>(h.flags.p + 1);
    unsigned long long *cnt = reinterpret_cast<unsigned long long *>(h.flags.p + 2);
    Prof prof(ctx, XLOG_HIP_KERNEL_HASH_INSERT, 24.0 * (double)n);
    unsigned long long *work = prof.work(1.0);
    const uint64_t waves = (n + WAVE - 1) / WAVE;
    const unsigned grid = grid_for(waves * WAVE, HB, std::min<unsigned>((unsigned)ctx->num_cus * 32, HS_MAX_BLOCKS));
    hipLaunchKernelGGL(k_hs_join_insert, dim3(grid), dim3(HB), 0, ctx->stream, a, view(h), out, cnt, limit, ovf,
                       work);
    XH_CHECK_HIP(hipGetLastError());
}

void hs_path_insert(Ctx *ctx, HashSet &h, const PathInsertArgs &a, uint64_t *out, uint64_t limit,
                    unsigned long long *count, unsigned long long *overflow) {
    if (!a.n) return;
    unsigned long long *ovf = overflow ? overflow : reinterpret_cast<unsigned long long *>(h.flags.p + 1);
    unsigned long long *cnt = count ? count : reinterpret_cast<unsigned long long *>(h.flags.p + 2);
    Prof prof(ctx, XLOG_HIP_KERNEL_HASH_INSERT, 0.0);  // bytes counted on the device (the row count may be there)
    unsigned long long *work = prof.work(1.0);
    const uint64_t waves = (a.n + WAVE - 1) / WAVE;
    const unsigned grid = grid_for(waves * WAVE, HB, std::min<unsigned>((unsigned)ctx->num_cus * 32, HS_MAX_BLOCKS));
    if (a.h2.table)
        hipLaunchKernelGGL(k_hs_path_insert<true>, dim3(grid), dim3(HB), 0, ctx->stream, a, view(h), out, cnt, limit,
                           ovf, work);
    else
        hipLaunchKernelGGL(k_hs_path_insert<false>, dim3(grid), dim3(HB), 0, ctx->stream, a, view(h), out, cnt, limit,
                           ovf, work);
    XH_CHECK_HIP(hipGetLastError());
}

void hs_insert_novel(Ctx *ctx, HashSet &h, const uint64_t *keys, uint64_t n, uint64_t *out, uint64_t limit,
                     int swap, unsigned long long *count, unsigned long long *overflow, const QueuedStep *q) {
    if (!n) return;
    unsigned long long *ovf = overflow ? overflow : reinterpret_cast<unsigned long long *>(h.flags.p + 1);
    unsigned long long *cnt = count ? count : reinterpret_cast<unsigned long long *>(h.flags.p + 2);
    Prof prof(ctx, XLOG_HIP_KERNEL_HASH_INSERT, 0.0);  // bytes counted on the device
    hipLaunchKernelGGL(k_hs_insert_novel, dim3(grid_blocks(ctx, n)), dim3(HB), 0, ctx->stream, keys, n, view(h), out,
                       cnt, limit, ovf, swap, q ? *q : QueuedStep(), prof.work(1.0));
    XH_CHECK_HIP(hipGetLastError());
}

uint64_t hs_collect(Ctx *ctx, const HashSet &h, uint64_t *out) {
    // the occupied slots in table order (a single-pass look-back selection), then the all-ones key
    Buf<uint64_t> cnt(ctx, 1);
    select_not_value(ctx, h.slots.p, h.cap, HS_EMPTY, out, cnt.p);
    hipLaunchKernelGGL(k_hs_append_allones, dim3(1), dim3(1), 0, ctx->stream,
                       reinterpret_cast<const unsigned int *>(h.flags.p), out, cnt.p);
    XH_CHECK_HIP(hipGetLastError());
    ctx->read_scalars(cnt.p, 1);
    return ctx->host_scalars[0];
}

}  // namespace xh
