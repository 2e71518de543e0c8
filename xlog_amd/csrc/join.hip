// Equi-join on one u32 key column for gfx950.
//
// Replaces the reference's bucketed-CSR hash join
// (hash_join_v2 / build_hash_table_v2 / hash_join_probe_v2,
//  crates/xlog-cuda/src/provider/relational.rs:2926-2992,4262-4625,
//  kernels/join.cu:131-252; pack_and_hash_keys, pack.cu:144-214) with:
//   build  - the build side arrives sorted by its key word (the high word of
//            the packed row), so every distinct key is one contiguous run.
//            One selection pass extracts (run key, run start); an
//            open-addressing table in HBM (16-byte slots holding key, run
//            length and run start, linear probing, Fibonacci hashing,
//            load <= 0.5) maps key -> run, so a probe row reads one slot and
//            then its run.  Keys are compared exactly, so colliding hashes
//            cannot produce matches (join_collision_test.rs:19-194).
//   probe  - two launches.  count: every probe row looks up its run, records
//            (run start, length) and a tile total is written.  emit: after a
//            scan of the tile totals, reading the recorded runs,
//            each wave expands its 64 rows' runs cooperatively: lane j of a
//            round writes output j, j+64, ... of the wave, found by a
//            6-step binary lifting over the per-row prefix in LDS, so
//            writes are contiguous across lanes and a hot key's long run is
//            shared by all lanes instead of serialising one thread.
//            The projection is fused into the emit.
#include "internal.hpp"

#include <algorithm>

namespace xh {

namespace {

constexpr int JB = 256;      // block
// Probe rows per thread (a tile is JB * JITEMS rows) and outputs per lane
// per expansion step of the emit.  Measured on MI355X over the C2 join
// (2^24 probe rows, 2.7e8 outputs): (rows, unroll) = (2, 4) 1.01 ms per emit,
// (4, 4) 1.03, (8, 4) 1.14, (16, 1) 1.42 -- small tiles with several payload
// loads in flight per lane beat deep per-thread lookup batches.
#ifndef XH_JITEMS
#define XH_JITEMS 2
#endif
#ifndef XH_EMIT_UNROLL
#define XH_EMIT_UNROLL 4
#endif
constexpr int JITEMS = XH_JITEMS;
constexpr int EMIT_UNROLL = XH_EMIT_UNROLL;
constexpr int JWAVES = JB / WAVE;
constexpr uint64_t tile_rows(int items) { return (uint64_t)JB * items; }

__device__ __forceinline__ uint64_t hash_slot(uint32_t key, int bits) {
    return (uint64_t)(((uint64_t)key * 0x9E3779B97F4A7C15ull) >> (64 - bits));
}

// Slot h = table[2h .. 2h+1]: (key << 32) | run length (0 = empty slot; a
// run is never empty), then the run start.
typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u64x2 load_slot(const unsigned long long *table, uint64_t h) {
    return *reinterpret_cast<const u64x2 *>(table + 2 * h);
}

__global__ void k_insert(const uint32_t *__restrict__ run_key, const uint64_t *__restrict__ run_start, uint64_t nruns,
                         unsigned long long *table, uint64_t mask, int bits) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < nruns; r += stride) {
        const uint32_t key = run_key[r];
        const uint64_t st = run_start[r], len = run_start[r + 1] - st;
        const unsigned long long v = ((unsigned long long)key << 32) | (unsigned long long)len;
        uint64_t h = hash_slot(key, bits);
        for (;;) {
            unsigned long long old = atomicCAS(&table[2 * h], 0ull, v);
            if (old == 0ull) {
                table[2 * h + 1] = st;  // read only by later launches
                break;
            }
            h = (h + 1) & mask;
        }
    }
}

// k_insert for a run list whose count is on the device (*d_nruns, at most
// runs_bound, which the table was sized for: at most half its slots fill)
// over sorted keys whose count is *d_n (the last run ends there); a raised
// stop ends it.
__global__ void k_insert_dev(const uint32_t *__restrict__ run_key, const uint64_t *__restrict__ run_start,
                             const uint64_t *d_nruns, uint64_t runs_bound, const uint64_t *d_n,
                             unsigned long long *table, uint64_t mask, int bits, const uint32_t *stop) {
    if (stop && *stop) return;
    const uint64_t nruns = *d_nruns < runs_bound ? *d_nruns : runs_bound, n = *d_n;
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < nruns; r += stride) {
        const uint32_t key = run_key[r];
        const uint64_t st = run_start[r], en = r + 1 < nruns ? run_start[r + 1] : n;
        const unsigned long long v = ((unsigned long long)key << 32) | (unsigned long long)(en - st);
        uint64_t h = hash_slot(key, bits);
        for (;;) {
            unsigned long long old = atomicCAS(&table[2 * h], 0ull, v);
            if (old == 0ull) {
                table[2 * h + 1] = st;  // read only by later launches
                break;
            }
            h = (h + 1) & mask;
        }
    }
}

__global__ void k_set_u64(uint64_t *p, uint64_t v) { *p = v; }
__global__ void k_max_run_len(const uint64_t *__restrict__ run_start, uint64_t nruns, unsigned long long *mx) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    unsigned long long m = 0;
    for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < nruns; r += stride)
        m = max(m, (unsigned long long)(run_start[r + 1] - run_start[r]));
    atomicMax(mx, m);
}

__device__ __forceinline__ bool lookup_run(const unsigned long long *__restrict__ table, uint64_t mask, int bits,
                                           uint32_t key, uint64_t *start, uint32_t *len) {
    uint64_t h = hash_slot(key, bits);
    for (;;) {
        const u64x2 s = load_slot(table, h);
        if (s.x == 0ull) return false;
        if ((uint32_t)(s.x >> 32) == key) {
            *start = s.y;
            *len = (uint32_t)s.x;
            return true;
        }
        h = (h + 1) & mask;
    }
}

struct ProbeArgs {
    const uint64_t *probe;
    uint64_t n;
    int pcol;  // 0: key = high word of the probe row, 1: low word
    const unsigned long long *table;  // 16-byte slots (load_slot)
    uint64_t mask;
    int bits;
    const uint32_t *payload;
    // optional row groups (see ProbeJob): gsel[i] = -1 plain row, -2 row
    // without output, g >= 0 row whose outputs are gsrc[gseg[2g] ..
    // gseg[2g] + gseg[2g + 1]) (finished output words)
    const int32_t *gsel;
    const uint64_t *gseg;
    const uint64_t *gsrc;
    // optional precomputed lookups (sort-merge join): run start and length
    // of every probe row; the table is not read when set
    const uint64_t *pre_start;
    const uint32_t *pre_cnt;
    // optional record of the count pass's lookups (read back by the emit as
    // pre_start / pre_cnt)
    uint64_t *rec_start;
    uint32_t *rec_cnt;
    // optional device-side row count (deferred count pass): when set, it
    // replaces n, which is then only the bound the grid was sized for
    const uint64_t *d_n;
    // optional profiling counter: the deferred count pass adds its real row count
    unsigned long long *work;
    // queued iterations: the stop flag (raised: the count writes zero tile
    // counts, the emit nothing) and the emit's output base on the device
    // (outputs go to out + *d_out_base).  With stop_code, a count pass whose
    // device row count is past its bound raises the flag with that code (its
    // own blocks then count at most the bound: the results are discarded).
    uint32_t *stop;
    const uint64_t *d_out_base;
    uint32_t stop_code;
    // optional output filter (EmitFilter), for two-column outputs of ids below 64 * fwords: an output
    // (x, z) is dropped when bit z of row x is set in fr (R's bit matrix, may be null) or in fseen (the
    // outputs already taken: the bit is claimed by an atomic OR); the others are appended to out0 at
    // positions taken from *fcount (positions at or past fcap are counted, not written)
    const uint64_t *fr;
    unsigned long long *fseen;
    unsigned long long *fcount;
    uint64_t fcap;
    uint32_t fwords;
};
// set in a row's start when its outputs come from gsrc
constexpr uint64_t GROUP_BIT = 1ull << 63;

// Lookups of N probe rows with their memory latencies overlapped: all first
// slots (and group selectors) are loaded together, the rare collision chains
// are walked after.  cnt[i] = 0 for rows with idx >= n.
template <int N>
__device__ __forceinline__ void lookup_batch(const ProbeArgs &a, const uint64_t *rows, uint64_t wbase, int lane,
                                             uint64_t *start, uint32_t *cnt) {
    // chunks of at most 8 rows keep the in-flight 16-byte slots within the
    // register budget of 4 waves per SIMD
    constexpr int C = N < 8 ? N : 8;
    static_assert(N % C == 0, "lookup chunking");
    if (a.pre_cnt) {  // block-uniform
#pragma unroll
        for (int r = 0; r < N; ++r) {
            const uint64_t idx = wbase + (uint64_t)r * WAVE + lane;
            const bool valid = idx < a.n;
            start[r] = valid ? a.pre_start[idx] : 0ull;
            cnt[r] = valid ? a.pre_cnt[idx] : 0u;
        }
        return;
    }
#pragma unroll
    for (int c0 = 0; c0 < N; c0 += C) {
        u64x2 slot[C];
        int32_t g[C];
#pragma unroll
        for (int q = 0; q < C; ++q) {
            const int r = c0 + q;
            const uint32_t key = a.pcol ? (uint32_t)rows[r] : (uint32_t)(rows[r] >> 32);
            const uint64_t idx = wbase + (uint64_t)r * WAVE + lane;
            const bool valid = idx < a.n;
            slot[q] = valid ? load_slot(a.table, hash_slot(key, a.bits)) : u64x2{0ull, 0ull};
            g[q] = (a.gsel && valid) ? a.gsel[idx] : -1;
        }
#pragma unroll
        for (int q = 0; q < C; ++q) {
            const int r = c0 + q;
            const uint32_t key = a.pcol ? (uint32_t)rows[r] : (uint32_t)(rows[r] >> 32);
            u64x2 s = slot[q];
            if (s.x != 0ull && (uint32_t)(s.x >> 32) != key) {  // rare: walk the collision chain
                uint64_t hh = hash_slot(key, a.bits);
                do {
                    hh = (hh + 1) & a.mask;
                    s = load_slot(a.table, hh);
                } while (s.x != 0ull && (uint32_t)(s.x >> 32) != key);
            }
            start[r] = s.x ? s.y : 0ull;
            cnt[r] = (uint32_t)s.x;  // 0 when the key has no run (empty slot)
            if (g[q] == -2) cnt[r] = 0;
            if (g[q] >= 0) {
                // without gseg the group outputs are not known yet: the head
                // counts zero here and k_group_fixup adds its group later
                start[r] = a.gseg ? (a.gseg[2 * g[q]] | GROUP_BIT) : 0ull;
                cnt[r] = a.gseg ? (uint32_t)a.gseg[2 * g[q] + 1] : 0u;
            }
        }
    }
}

template <int ITEMS>
__device__ __forceinline__ void probe_count_tile(const ProbeArgs &a, uint64_t tile, uint64_t *__restrict__ tile_cnt,
                                                 uint64_t *s_part, int tid, int lane, int wave) {
    const uint64_t wbase = tile * tile_rows(ITEMS) + (uint64_t)wave * (ITEMS * WAVE);
    uint64_t rows[ITEMS];
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) {
        uint64_t idx = wbase + (uint64_t)r * WAVE + lane;
        rows[r] = idx < a.n ? a.probe[idx] : 0ull;
    }
    uint64_t starts[ITEMS];
    uint32_t cnts[ITEMS];
    lookup_batch<ITEMS>(a, rows, wbase, lane, starts, cnts);
    if (a.rec_cnt) {  // block-uniform
#pragma unroll
        for (int r = 0; r < ITEMS; ++r) {
            const uint64_t idx = wbase + (uint64_t)r * WAVE + lane;
            if (idx < a.n) {
                a.rec_start[idx] = starts[r];
                a.rec_cnt[idx] = cnts[r];
            }
        }
    }
    uint64_t acc = 0;
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) acc += cnts[r];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, WAVE);
    if (lane == 0) s_part[wave] = acc;
    __syncthreads();
    if (tid == 0) {
        uint64_t t = 0;
        for (int w = 0; w < JWAVES; ++w) t += s_part[w];
        tile_cnt[tile] = t;
    }
}

// One tile per block, or, with a device row count (a.d_n; a.n is then the
// bound), a grid of a few blocks per CU striding over the bound's tiles: the
// tiles past the real rows count zero at the cost of one store each.
template <int ITEMS>
__global__ __launch_bounds__(JB) void k_probe_count(ProbeArgs a, uint64_t *__restrict__ tile_cnt) {
    __shared__ uint64_t s_part[JWAVES];
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    if (!a.d_n) {
        probe_count_tile<ITEMS>(a, blockIdx.x, tile_cnt, s_part, tid, lane, wave);
        return;
    }
    if (a.stop && *a.stop) return;  // a stopped queue: nothing reads these counts
    const uint64_t bound_tiles = (a.n + tile_rows(ITEMS) - 1) / tile_rows(ITEMS);
    if (*a.d_n > a.n && a.stop_code && blockIdx.x == 0 && tid == 0) atomicCAS(a.stop, 0u, a.stop_code);
    if (*a.d_n < a.n) a.n = *a.d_n;
    if (a.work && blockIdx.x == 0 && tid == 0) atomicAdd(a.work, (unsigned long long)a.n);
    for (uint64_t t = blockIdx.x; t < bound_tiles; t += gridDim.x) {
        if (t * tile_rows(ITEMS) >= a.n) {
            if (tid == 0) tile_cnt[t] = 0;
            continue;
        }
        probe_count_tile<ITEMS>(a, t, tile_cnt, s_part, tid, lane, wave);
        __syncthreads();  // s_part is reused by the next tile
    }
}

// Output spec: up to 4 selected values among v0 = probe.c0, v1 = probe.c1,
// v2 = build key, v3 = build payload, packed per the relation layout.
struct OutSpec {
    int arity;   // 1..4
    int oc[4];
};
__device__ __forceinline__ void make_words(const OutSpec &o, const uint32_t v[4], uint64_t *w0, uint64_t *w1) {
    if (o.arity == 1) {
        *w0 = v[o.oc[0]];
        *w1 = 0;
        return;
    }
    *w0 = ((uint64_t)v[o.oc[0]] << 32) | v[o.oc[1]];
    if (o.arity == 3) *w1 = (uint64_t)v[o.oc[2]] << 32;
    else if (o.arity == 4) *w1 = ((uint64_t)v[o.oc[2]] << 32) | v[o.oc[3]];
    else *w1 = 0;
}

// One output per lane through the filter (lanes with live = false only take
// part in the wave's append): the wave's kept outputs take consecutive
// positions from one atomic add.
__device__ __forceinline__ void filter_append(const ProbeArgs &a, bool live, uint64_t w, uint64_t *__restrict__ out,
                                              int lane) {
    bool keep = false;
    if (live) {
        const uint64_t x = w >> 32;
        const uint32_t z = (uint32_t)w;
        const uint64_t idx = x * a.fwords + (z >> 6);
        const unsigned long long m = 1ull << (z & 63u);
        // (a plain read first: a bit once set stays set, so only a clear bit needs the atomic)
        if (!(a.fr && (a.fr[idx] & m)) && !(a.fseen[idx] & m)) keep = !(atomicOr(&a.fseen[idx], m) & m);
    }
    const uint64_t bal = __ballot(keep);
    if (!bal) return;
    const int leader = __ffsll((unsigned long long)bal) - 1;
    unsigned long long base = 0;
    if (lane == leader) base = atomicAdd(a.fcount, (unsigned long long)__popcll(bal));
    base = __shfl(base, leader, WAVE);
    if (keep) {
        const uint64_t pos = base + (uint64_t)__popcll(bal & ((1ull << lane) - 1ull));
        if (pos < a.fcap) out[pos] = w;
    }
}

// The outputs of one probe tile (k_probe_emit).
struct EmitSmem {
    uint64_t wtot[JWAVES];
    uint64_t ex[JWAVES][WAVE + 1];
    uint64_t row[JWAVES][WAVE];
    uint64_t st[JWAVES][WAVE];
};
template <int ITEMS, bool FILT = false>
__device__ __forceinline__ void probe_emit_tile(const ProbeArgs &a, const uint64_t *__restrict__ tile_off, uint64_t t0,
                                                uint64_t tile, const OutSpec &spec, uint64_t *__restrict__ out0,
                                                uint64_t *__restrict__ out1, EmitSmem &sm, int tid, int lane,
                                                int wave) {
    uint64_t *s_wtot = sm.wtot;
    auto &s_ex = sm.ex;
    auto &s_row = sm.row;
    auto &s_st = sm.st;
    const uint64_t wbase = tile * tile_rows(ITEMS) + (uint64_t)wave * (ITEMS * WAVE);

    // pass 1 over this wave's rows: all ITEMS lookups issued together (their
    // latencies overlap) and kept in registers for the expansion
    uint64_t rows[ITEMS], starts[ITEMS];
    uint32_t cnts[ITEMS];
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) {
        uint64_t idx = wbase + (uint64_t)r * WAVE + lane;
        rows[r] = idx < a.n ? a.probe[idx] : 0ull;
    }
    lookup_batch<ITEMS>(a, rows, wbase, lane, starts, cnts);
    uint64_t acc = 0;
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) acc += cnts[r];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, WAVE);
    if (lane == 0) s_wtot[wave] = acc;
    __syncthreads();
    uint64_t base = tile_off[tile] - tile_off[t0];
    for (int w = 0; w < wave; ++w) base += s_wtot[w];

    // pass 2: expand round by round
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) {
        const uint64_t row = rows[r], st = starts[r], c = cnts[r];
        uint64_t x = c;
#pragma unroll
        for (int o = 1; o < WAVE; o <<= 1) {
            uint64_t t = __shfl_up(x, o, WAVE);
            if (lane >= o) x += t;
        }
        uint64_t total = __shfl(x, WAVE - 1, WAVE);
        if (total == 0) continue;
        s_ex[wave][lane] = x - c;
        s_row[wave][lane] = row;
        s_st[wave][lane] = st;
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // EMIT_UNROLL outputs per lane per step, so that their payload loads
        // are in flight together
        for (uint64_t j0 = lane; j0 < total; j0 += EMIT_UNROLL * WAVE) {
            uint64_t prow[EMIT_UNROLL], bpos[EMIT_UNROLL];
            uint32_t pay[EMIT_UNROLL];
            uint64_t gw[EMIT_UNROLL];
            // row of output j: the largest s with ex[s] <= j (ex[0] = 0 and ex
            // is non-decreasing, so an empty row resolves to the next
            // non-empty one), by binary lifting in 6 fixed steps; the
            // EMIT_UNROLL searches advance level by level, so their LDS reads
            // overlap instead of forming EMIT_UNROLL dependent chains
            int lo[EMIT_UNROLL];
#pragma unroll
            for (int u = 0; u < EMIT_UNROLL; ++u) lo[u] = 0;
#pragma unroll
            for (int step = WAVE / 2; step > 0; step >>= 1) {
#pragma unroll
                for (int u = 0; u < EMIT_UNROLL; ++u) {
                    const uint64_t j = j0 + (uint64_t)u * WAVE;
                    lo[u] += s_ex[wave][lo[u] + step] <= j ? step : 0;  // lo[u] + step <= WAVE - 1
                }
            }
#pragma unroll
            for (int u = 0; u < EMIT_UNROLL; ++u) {
                const uint64_t j = j0 + (uint64_t)u * WAVE;
                prow[u] = s_row[wave][lo[u]];
                bpos[u] = s_st[wave][lo[u]] + (j - s_ex[wave][lo[u]]);
                const bool live = j < total;
                const bool grp = (bpos[u] & GROUP_BIT) != 0;
                pay[u] = (live && !grp && a.payload) ? a.payload[bpos[u]] : 0u;
                gw[u] = (live && grp) ? a.gsrc[bpos[u] & ~GROUP_BIT] : 0ull;
            }
            if (FILT) {  // filtered two-column outputs, appended
#pragma unroll
                for (int u = 0; u < EMIT_UNROLL; ++u) {
                    const uint64_t j = j0 + (uint64_t)u * WAVE;
                    uint64_t w0 = 0, w1;
                    if (j < total) {
                        uint32_t v[4];
                        v[0] = (uint32_t)(prow[u] >> 32);
                        v[1] = (uint32_t)prow[u];
                        v[2] = a.pcol ? (uint32_t)prow[u] : (uint32_t)(prow[u] >> 32);
                        v[3] = pay[u];
                        make_words(spec, v, &w0, &w1);
                    }
                    filter_append(a, j < total, w0, out0, lane);
                }
                continue;
            }
#pragma unroll
            for (int u = 0; u < EMIT_UNROLL; ++u) {
                const uint64_t j = j0 + (uint64_t)u * WAVE;
                if (j >= total) break;
                uint64_t w0, w1;
                if (bpos[u] & GROUP_BIT) {
                    w0 = gw[u];
                    w1 = 0;
                } else {
                    uint32_t v[4];
                    v[0] = (uint32_t)(prow[u] >> 32);
                    v[1] = (uint32_t)prow[u];
                    v[2] = a.pcol ? (uint32_t)prow[u] : (uint32_t)(prow[u] >> 32);
                    v[3] = pay[u];
                    make_words(spec, v, &w0, &w1);
                }
                out0[base + j] = w0;
                if (out1) out1[base + j] = w1;
            }
        }
        base += total;
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
}

// Emits the outputs of tiles [t0, t0 + gridDim.x); output index 0 is the
// first output of tile t0.  With a device row count (a.d_n; a.n is then the
// bound, t0 is 0) a grid of a few blocks per CU strides over the real tiles;
// a.d_out_base then offsets the output.
template <int ITEMS, bool FILT = false>
__global__ __launch_bounds__(JB) void k_probe_emit(ProbeArgs a, const uint64_t *__restrict__ tile_off, uint64_t t0,
                                                   OutSpec spec, uint64_t *__restrict__ out0,
                                                   uint64_t *__restrict__ out1) {
    __shared__ EmitSmem sm;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    if (!a.d_n) {
        probe_emit_tile<ITEMS, FILT>(a, tile_off, t0, t0 + blockIdx.x, spec, out0, out1, sm, tid, lane, wave);
        return;
    }
    if (a.stop && *a.stop) return;
    if (*a.d_n < a.n) a.n = *a.d_n;
    if (a.d_out_base) {
        const uint64_t ob = *a.d_out_base;
        out0 += ob;
        if (out1) out1 += ob;
    }
    const uint64_t tiles = (a.n + tile_rows(ITEMS) - 1) / tile_rows(ITEMS);
    for (uint64_t t = blockIdx.x; t < tiles; t += gridDim.x) {
        probe_emit_tile<ITEMS, FILT>(a, tile_off, 0, t, spec, out0, out1, sm, tid, lane, wave);
        __syncthreads();  // the shared arrays are reused by the next tile
    }
}

// Sort-merge join lookup (reference sort_merge_join_v2_inner_u32_1key,
// relational.rs:3401-3571, kernels/join.cu:665-712, which binary-searches the
// sorted right keys once per left row).  The left rows, sorted by key, are
// merged with the sorted distinct run keys of the right side along the merge
// path: a tile is 2048 consecutive items of the merged sequence, whatever mix
// of left rows and runs they are, so every block does the same work however
// the keys are skewed; runs go first on equal keys, so a left row's match is
// the last run merged before it, when that run has the row's key.  Output per
// left row: run start and length (0 without a match), for the probe's count
// and emit, which spread each row's run over the lanes of a wave.
constexpr int SMJ_BLOCK = 256, SMJ_ITEMS = 8, SMJ_TILE = SMJ_BLOCK * SMJ_ITEMS;

// number of runs among the first d items of the merge (runs first on ties)
template <typename RK, typename LK>
__device__ __forceinline__ uint64_t smj_path(RK rkey, uint64_t nr, LK lkey, uint64_t nl, uint64_t d) {
    uint64_t lo = d > nl ? d - nl : 0, hi = d < nr ? d : nr;
    while (lo < hi) {
        const uint64_t mid = (lo + hi) >> 1;
        if (rkey(mid) <= lkey(d - mid - 1)) lo = mid + 1; else hi = mid;
    }
    return lo;
}

// split[t] = smj_path at diagonal min(t * SMJ_TILE, nl + nr), one thread per
// tile boundary (all tiles' binary searches side by side, not two dependent
// chains at the start of every lookup block)
__global__ void k_smj_partition(const uint64_t *__restrict__ l, uint64_t nl, int pcol,
                                const uint32_t *__restrict__ run_key, uint64_t nr, uint64_t tiles,
                                uint64_t *__restrict__ split) {
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t > tiles) return;
    auto lkey_g = [&](uint64_t i) { const uint64_t r = l[i]; return pcol ? (uint32_t)r : (uint32_t)(r >> 32); };
    auto rkey_g = [&](uint64_t i) { return run_key[i]; };
    const uint64_t total = nl + nr, d = t * SMJ_TILE < total ? t * SMJ_TILE : total;
    split[t] = smj_path(rkey_g, nr, lkey_g, nl, d);
}

__global__ __launch_bounds__(SMJ_BLOCK) void k_smj_lookup(const uint64_t *__restrict__ l, uint64_t nl, int pcol,
                                                          const uint32_t *__restrict__ run_key,
                                                          const uint64_t *__restrict__ run_start, uint64_t nr,
                                                          const uint64_t *__restrict__ split,
                                                          uint64_t *__restrict__ start, uint32_t *__restrict__ cnt) {
    __shared__ uint32_t s_key[SMJ_TILE];  // the tile's runs, then its left rows
    __shared__ uint64_t s_split[2];
    const int tid = threadIdx.x;
    auto lkey_g = [&](uint64_t i) { const uint64_t r = l[i]; return pcol ? (uint32_t)r : (uint32_t)(r >> 32); };
    const uint64_t total = nl + nr;
    const uint64_t d0 = (uint64_t)blockIdx.x * SMJ_TILE;
    const uint64_t d1 = d0 + SMJ_TILE < total ? d0 + SMJ_TILE : total;
    if (tid < 2) s_split[tid] = split[blockIdx.x + tid];
    __syncthreads();
    // (sorted inputs give monotone splits; the clamp keeps a tile's ranges inside both inputs and LDS otherwise)
    const uint64_t r0 = s_split[0];
    uint64_t r1 = s_split[1];
    {
        const uint64_t lo1 = d1 > nl && d1 - nl > r0 ? d1 - nl : r0;
        const uint64_t hi1 = r0 + (d1 - d0) < nr ? r0 + (d1 - d0) : nr;
        r1 = r1 < lo1 ? lo1 : (r1 > hi1 ? hi1 : r1);
    }
    const uint32_t len = (uint32_t)(d1 - d0), lr = (uint32_t)(r1 - r0), ll = len - lr;
    const uint64_t l0 = d0 - r0;
    batched_copy<SMJ_BLOCK, SMJ_ITEMS>(
        len, tid, [&](uint32_t i) { return i < lr ? run_key[r0 + i] : lkey_g(l0 + (i - lr)); },
        [&](uint32_t i, uint32_t v) { s_key[i] = v; });
    __syncthreads();
    const uint32_t *sr = s_key, *sl = s_key + lr;
    const uint32_t td = (uint32_t)tid * SMJ_ITEMS;
    if (td >= len) return;
    auto rkey_s = [&](uint64_t i) { return sr[i]; };
    auto lkey_s = [&](uint64_t i) { return sl[i]; };
    uint32_t ir = (uint32_t)smj_path(rkey_s, lr, lkey_s, ll, td);
    uint32_t il = td - ir;
    // the run merged last before this thread's first item
    bool have = r0 + ir > 0;
    uint64_t cur = have ? r0 + ir - 1 : 0;
    uint32_t cur_key = have ? (ir > 0 ? sr[ir - 1] : run_key[r0 - 1]) : 0u;
    const uint32_t end = td + SMJ_ITEMS < len ? td + SMJ_ITEMS : len;
    for (uint32_t t = td; t < end; ++t) {
        const bool take_r = il >= ll || (ir < lr && sr[ir] <= sl[il]);
        if (take_r) {
            cur = r0 + ir;
            cur_key = sr[ir];
            have = true;
            ++ir;
        } else {
            const uint64_t row = l0 + il;
            const bool hit = have && cur_key == sl[il];
            const uint64_t st = hit ? run_start[cur] : 0ull;
            start[row] = st;
            cnt[row] = hit ? (uint32_t)(run_start[cur + 1] - st) : 0u;
            ++il;
        }
    }
}

// semi / anti: flag = key found (semi) or not found (anti)
__global__ void k_match_flags(ProbeArgs a, int want, uint8_t *__restrict__ flags) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += stride) {
        uint64_t row = a.probe[i];
        uint32_t key = a.pcol ? (uint32_t)row : (uint32_t)(row >> 32);
        uint64_t st;
        uint32_t len;
        bool hit = lookup_run(a.table, a.mask, a.bits, key, &st, &len);
        flags[i] = (uint8_t)(hit == (want != 0));
    }
}

// two keys: the key word found and the other word among the run's payloads
// (which ascend inside the run: an index on the first column of a sorted
// relation)
__global__ void k_match2_flags(ProbeArgs a, uint8_t *__restrict__ flags) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += stride) {
        const uint64_t row = a.probe[i];
        const uint32_t key = a.pcol ? (uint32_t)row : (uint32_t)(row >> 32);
        const uint32_t other = a.pcol ? (uint32_t)(row >> 32) : (uint32_t)row;
        uint64_t st;
        uint32_t len;
        bool found = false;
        if (lookup_run(a.table, a.mask, a.bits, key, &st, &len)) {
            uint64_t lo = st, hi = st + len;
            while (lo < hi) {
                const uint64_t mid = lo + ((hi - lo) >> 1);
                if (a.payload[mid] < other) lo = mid + 1; else hi = mid;
            }
            found = lo < st + len && a.payload[lo] == other;
        }
        flags[i] = (uint8_t)found;
    }
}

// Triangle existence (wcoj_triangle_flags): row i of `mask` holds (u, v), or
// (v, u) with mask_swap; it is kept when the run of u in P and the run of v in
// Q share a payload value w.  Both runs' payloads ascend, so the shorter run's
// values are searched in the longer one, each search starting where the last
// ended (a value past the longer run's end ends the row).
__global__ void k_wcoj_triangle(const uint64_t *__restrict__ mask, uint64_t n, int mask_swap,
                                const unsigned long long *__restrict__ pt, uint64_t pmask, int pbits,
                                const uint32_t *__restrict__ ppay, const unsigned long long *__restrict__ qt,
                                uint64_t qmask, int qbits, const uint32_t *__restrict__ qpay,
                                uint8_t *__restrict__ flags) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t row = mask[i];
        const uint32_t u = mask_swap ? (uint32_t)row : (uint32_t)(row >> 32);
        const uint32_t v = mask_swap ? (uint32_t)(row >> 32) : (uint32_t)row;
        uint64_t sp = 0, sq = 0;
        uint32_t lp = 0, lq = 0;
        bool found = false;
        if (lookup_run(pt, pmask, pbits, u, &sp, &lp) && lookup_run(qt, qmask, qbits, v, &sq, &lq)) {
            const uint32_t *a = ppay + sp, *b = qpay + sq;  // a: the shorter run
            uint32_t la = lp, lb = lq;
            if (la > lb) {
                const uint32_t *t = a;
                a = b;
                b = t;
                const uint32_t tl = la;
                la = lb;
                lb = tl;
            }
            uint32_t lo = 0;
            for (uint32_t k = 0; k < la && !found; ++k) {
                const uint32_t x = a[k];
                uint32_t hi = lb;
                while (lo < hi) {
                    const uint32_t mid = lo + ((hi - lo) >> 1);
                    if (b[mid] < x) lo = mid + 1; else hi = mid;
                }
                if (lo == lb) break;
                found = b[lo] == x;
            }
        }
        flags[i] = (uint8_t)found;
    }
}

}  // namespace

// Runs of the high word of sorted keys [0, n), n = *d_n when d_n is set
// (then n_bound sizes the buffers): key and start per run, the run count to
// *d_nruns.  build_run_index_finish builds the table once the host knows the
// run count and n.
void build_run_index_async(Ctx *ctx, const uint64_t *sorted_keys, uint64_t n_bound, const uint64_t *d_n,
                           RunScratch &rs, uint64_t *d_nruns) {
    rs.run_key = Buf<uint32_t>(ctx, n_bound ? n_bound : 1);
    rs.run_start = Buf<uint64_t>(ctx, n_bound + 1);
    select_runs(ctx, sorted_keys, n_bound, rs.run_key.p, rs.run_start.p, d_nruns, d_n);
}
void build_run_index_finish(Ctx *ctx, RunScratch &rs, uint64_t nruns, uint64_t n, RunIndex &ix) {
    ix.nruns = nruns;
    XH_REQUIRE(ix.nruns < 0xFFFFFFFFull, XLOG_HIP_CAPACITY_OVERFLOW, "join build: too many distinct keys");
    hipLaunchKernelGGL(k_set_u64, dim3(1), dim3(1), 0, ctx->stream, rs.run_start.p + ix.nruns, n);
    if (n >= (1ull << 32) && ix.nruns) {  // a slot holds a 32-bit run length
        Buf<unsigned long long> mx(ctx, 1);
        fill_u64(ctx, reinterpret_cast<uint64_t *>(mx.p), 0ull, 1);
        hipLaunchKernelGGL(k_max_run_len, dim3(grid_for(ix.nruns, 256, 16384)), dim3(256), 0, ctx->stream,
                           rs.run_start.p, ix.nruns, mx.p);
        XH_CHECK_HIP(hipGetLastError());
        ctx->read_scalars(mx.p, 1);
        XH_REQUIRE(ctx->host_scalars[0] < (1ull << 32), XLOG_HIP_CAPACITY_OVERFLOW,
                   "join build: a key with 2^32 or more rows");
    }
    XH_CHECK_HIP(hipGetLastError());
    int bits = 10;
    while ((1ull << bits) < 2 * ix.nruns) ++bits;
    uint64_t slots = 1ull << bits;
    ix.table = Buf<unsigned long long>(ctx, 2 * slots);
    ix.table_mask = slots - 1;
    fill_u64(ctx, reinterpret_cast<uint64_t *>(ix.table.p), 0ull, 2 * slots);
    if (ix.nruns)
        hipLaunchKernelGGL(k_insert, dim3(grid_for(ix.nruns, 256, 16384)), dim3(256), 0, ctx->stream, rs.run_key.p,
                           rs.run_start.p, ix.nruns, ix.table.p, ix.table_mask, bits);
    XH_CHECK_HIP(hipGetLastError());
}
void run_index_insert_dev(Ctx *ctx, const uint32_t *run_key, const uint64_t *run_start, const uint64_t *d_nruns,
                          uint64_t runs_bound, const uint64_t *d_n, RunIndex &ix, const uint32_t *stop) {
    const uint64_t slots = ix.table_mask + 1;
    XH_REQUIRE(slots >= 2 * runs_bound, XLOG_HIP_INVALID_ARG, "run index: table smaller than twice its runs");
    fill_u64(ctx, reinterpret_cast<uint64_t *>(ix.table.p), 0ull, 2 * slots);
    if (!runs_bound) return;
    hipLaunchKernelGGL(k_insert_dev, dim3(persistent_grid(ctx, (runs_bound + 255) / 256, 8)), dim3(256), 0, ctx->stream,
                       run_key, run_start, d_nruns, runs_bound, d_n, ix.table.p, ix.table_mask, __builtin_ctzll(slots), stop);
    XH_CHECK_HIP(hipGetLastError());
}
void build_run_index(Ctx *ctx, const uint64_t *sorted_keys, uint64_t n, RunIndex &ix) {
    RunScratch rs;
    Buf<uint64_t> cnt(ctx, 1);
    build_run_index_async(ctx, sorted_keys, n, nullptr, rs, cnt.p);
    ctx->read_scalars(cnt.p, 1);
    build_run_index_finish(ctx, rs, ctx->host_scalars[0], n, ix);
}

static int table_bits(const RunIndex &ix) {
    int bits = 0;
    while ((1ull << bits) < ix.table_mask + 1) ++bits;
    return bits;
}

static ProbeArgs probe_args(const ProbeJob &job) {
    const RunIndex &ix = *job.ix;
    return ProbeArgs{job.probe, job.n, job.pcol, ix.table.p, ix.table_mask, table_bits(ix), job.payload, job.gsel,
                     job.gseg, job.gsrc, job.pre_start, job.pre_cnt, nullptr, nullptr};
}

uint64_t probe_prepare(Ctx *ctx, ProbeJob &job) {
    job.items = JITEMS;
    job.tiles = (job.n + tile_rows(job.items) - 1) / tile_rows(job.items);
    job.total = 0;
    if (job.n == 0 || job.ix->nruns == 0) return 0;
    XH_REQUIRE(job.tiles < (1ull << 31), XLOG_HIP_CAPACITY_OVERFLOW, "join probe: input too large");
    ProbeArgs a = probe_args(job);
    job.toff = Buf<uint64_t>(ctx, job.tiles + 1);
    if (!job.pre_cnt && job.record_lookups) {
        // the emit then reads each row's run from these arrays instead of
        // repeating the hash-table lookup
        job.rec_start = Buf<uint64_t>(ctx, job.n);
        job.rec_cnt = Buf<uint32_t>(ctx, job.n);
        a.rec_start = job.rec_start.p;
        a.rec_cnt = job.rec_cnt.p;
    }
    {
        // probe row + one 16-byte slot per row, + the 12-byte record when kept
        Prof prof(ctx, XLOG_HIP_KERNEL_PROBE_COUNT, (a.rec_cnt ? 36.0 : (job.pre_cnt ? 20.0 : 24.0)) * (double)job.n);
        hipLaunchKernelGGL(k_probe_count<JITEMS>, dim3((unsigned)job.tiles), dim3(JB), 0, ctx->stream, a,
                           job.toff.p);
        XH_CHECK_HIP(hipGetLastError());
    }
    scan_u64_inplace(ctx, job.toff.p, job.tiles, job.toff.p + job.tiles);
    ctx->read_scalars(job.toff.p + job.tiles, 1);
    job.total = ctx->host_scalars[0];
    XH_REQUIRE(job.total < SCAN64_EXACT, XLOG_HIP_CAPACITY_OVERFLOW,
               "join probe: " + std::to_string(job.total) + " output rows");
    if (a.rec_cnt) {
        job.pre_start = job.rec_start.p;
        job.pre_cnt = job.rec_cnt.p;
    }
    return job.total;
}

// The count pass and the tile scan for a probe whose row count is still on
// the device (*d_n <= n_bound): the grid, the tile offsets and the recorded
// lookups are sized for n_bound; nothing is read back.  probe_finish then
// takes the row count and the total (read back by the caller together with
// whatever else it needs: d_total() points at the total).
void probe_prepare_deferred(Ctx *ctx, ProbeJob &job, uint64_t n_bound, const uint64_t *d_n, uint32_t *stop,
                            uint32_t stop_code) {
    job.items = JITEMS;
    job.n = n_bound;
    job.tiles = (n_bound + tile_rows(job.items) - 1) / tile_rows(job.items);
    job.total = 0;
    XH_REQUIRE(job.tiles < (1ull << 31), XLOG_HIP_CAPACITY_OVERFLOW, "join probe: input too large");
    job.toff = Buf<uint64_t>(ctx, job.tiles + 1);
    if (n_bound == 0 || job.ix->nruns == 0) {
        fill_u64(ctx, job.toff.p, 0ull, job.tiles + 1);
        return;
    }
    ProbeArgs a = probe_args(job);
    a.d_n = d_n;
    a.stop = stop;
    a.stop_code = stop_code;
    XH_REQUIRE(!job.pre_cnt && job.record_lookups, XLOG_HIP_INVALID_ARG, "deferred probe: recorded lookups only");
    job.rec_start = Buf<uint64_t>(ctx, n_bound);
    job.rec_cnt = Buf<uint32_t>(ctx, n_bound);
    a.rec_start = job.rec_start.p;
    a.rec_cnt = job.rec_cnt.p;
    {
        Prof prof(ctx, XLOG_HIP_KERNEL_PROBE_COUNT, 0.0);
        a.work = prof.work(36.0);  // 36 B per real row, counted on the device
        hipLaunchKernelGGL(k_probe_count<JITEMS>, dim3(persistent_grid(ctx, job.tiles, 16)), dim3(JB), 0, ctx->stream,
                           a, job.toff.p);
        XH_CHECK_HIP(hipGetLastError());
    }
    // tiles past the real rows hold zero counts
    scan_u64_inplace(ctx, job.toff.p, job.tiles, job.toff.p + job.tiles, stop);
}

void probe_emit_dev(Ctx *ctx, const ProbeJob &job, const uint64_t *d_n, const int oc[4], uint64_t *out,
                    const uint64_t *d_out_base, uint32_t *stop, const EmitFilter *filter) {
    if (job.n == 0 || job.tiles == 0 || !job.rec_cnt.p) return;  // nothing can match (see probe_prepare_deferred)
    ProbeArgs a = probe_args(job);
    a.pre_start = job.rec_start.p;  // the count pass's recorded lookups
    a.pre_cnt = job.rec_cnt.p;
    a.d_n = d_n;
    a.stop = stop;
    a.d_out_base = d_out_base;
    if (filter) {
        XH_REQUIRE(!d_out_base && filter->seen && filter->count && filter->words, XLOG_HIP_INVALID_ARG,
                   "filtered probe emit: appended output only");
        a.fr = filter->rbits;
        a.fseen = reinterpret_cast<unsigned long long *>(filter->seen);
        a.fcount = reinterpret_cast<unsigned long long *>(filter->count);
        a.fcap = filter->cap;
        a.fwords = filter->words;
    }
    OutSpec spec{2, {oc[0], oc[1], oc[2], oc[3]}};
    // per probe row its record (20 B with the row) and per match 12 B, counted on the device
    Prof prof(ctx, XLOG_HIP_KERNEL_PROBE_EMIT, 0.0);
    add_work_rows(ctx, prof.work(1.0), d_n, job.n, 20, job.toff.p + job.tiles, ~0ull, 12, nullptr, stop);
    if (filter)
        hipLaunchKernelGGL((k_probe_emit<JITEMS, true>), dim3(persistent_grid(ctx, job.tiles, 16)), dim3(JB), 0,
                           ctx->stream, a, job.toff.p, 0ull, spec, out, nullptr);
    else
        hipLaunchKernelGGL(k_probe_emit<JITEMS>, dim3(persistent_grid(ctx, job.tiles, 16)), dim3(JB), 0, ctx->stream,
                           a, job.toff.p, 0ull, spec, out, nullptr);
    XH_CHECK_HIP(hipGetLastError());
}
void probe_finish(ProbeJob &job, uint64_t n, uint64_t total) {
    XH_REQUIRE(total < SCAN64_EXACT, XLOG_HIP_CAPACITY_OVERFLOW, "join probe: " + std::to_string(total) + " output rows");
    job.n = n;
    job.tiles = (n + tile_rows(job.items) - 1) / tile_rows(job.items);
    job.total = total;
    if (job.rec_cnt.p) {
        job.pre_start = job.rec_start.p;
        job.pre_cnt = job.rec_cnt.p;
    }
}

// The count pass alone (tile counts in job.toff[0..tiles), lookups recorded),
// for a caller that adds to the counts before probe_scan_async.  With gsel
// set and gseg null, group heads count zero (see k_group_fixup).
void probe_count_only(Ctx *ctx, ProbeJob &job) {
    job.items = JITEMS;
    job.tiles = (job.n + tile_rows(job.items) - 1) / tile_rows(job.items);
    job.total = 0;
    XH_REQUIRE(job.tiles < (1ull << 31), XLOG_HIP_CAPACITY_OVERFLOW, "join probe: input too large");
    XH_REQUIRE(job.record_lookups && !job.pre_cnt, XLOG_HIP_INVALID_ARG, "count-only probe: recorded lookups only");
    job.toff = Buf<uint64_t>(ctx, job.tiles + 1);
    if (job.n == 0) return;
    if (job.ix->nruns == 0) {
        fill_u64(ctx, job.toff.p, 0ull, job.tiles + 1);
        job.rec_start = Buf<uint64_t>(ctx, job.n);
        job.rec_cnt = Buf<uint32_t>(ctx, job.n);
        fill_u64(ctx, job.rec_start.p, 0ull, job.n);
        fill_u32(ctx, job.rec_cnt.p, 0u, job.n);
        return;
    }
    ProbeArgs a = probe_args(job);
    job.rec_start = Buf<uint64_t>(ctx, job.n);
    job.rec_cnt = Buf<uint32_t>(ctx, job.n);
    a.rec_start = job.rec_start.p;
    a.rec_cnt = job.rec_cnt.p;
    Prof prof(ctx, XLOG_HIP_KERNEL_PROBE_COUNT, 36.0 * (double)job.n);
    hipLaunchKernelGGL(k_probe_count<JITEMS>, dim3((unsigned)job.tiles), dim3(JB), 0, ctx->stream, a, job.toff.p);
    XH_CHECK_HIP(hipGetLastError());
}

namespace {
// Group heads of a count pass run without gseg: each head's recorded run
// becomes its group's finished words and its tile count grows by their number.
__global__ void k_group_fixup(const uint64_t *__restrict__ hpos, const uint64_t *__restrict__ gseg, uint64_t nh,
                              uint64_t *__restrict__ rec_start, uint32_t *__restrict__ rec_cnt,
                              unsigned long long *tile_cnt, uint64_t rows_per_tile) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t g = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; g < nh; g += stride) {
        const uint64_t p = hpos[g], st = gseg[2 * g], c = gseg[2 * g + 1];
        rec_start[p] = st | GROUP_BIT;
        rec_cnt[p] = (uint32_t)c;
        if (c) atomicAdd(tile_cnt + p / rows_per_tile, (unsigned long long)c);
    }
}
}  // namespace

void probe_group_fixup(Ctx *ctx, ProbeJob &job, const uint64_t *hpos, const uint64_t *gseg, uint64_t nh) {
    if (!nh || !job.n) return;
    hipLaunchKernelGGL(k_group_fixup, dim3(grid_for(nh, 256, 4096)), dim3(256), 0, ctx->stream, hpos, gseg, nh,
                       job.rec_start.p, job.rec_cnt.p, reinterpret_cast<unsigned long long *>(job.toff.p),
                       tile_rows(job.items));
    XH_CHECK_HIP(hipGetLastError());
}

// The tile scan of a count-only probe; the total lands at job.toff.p[job.tiles]
// (finish with probe_finish once the host has read it).
void probe_scan_async(Ctx *ctx, ProbeJob &job) {
    if (!job.n) return;
    scan_u64_inplace(ctx, job.toff.p, job.tiles, job.toff.p + job.tiles);
}

std::vector<uint64_t> probe_tile_offsets(Ctx *ctx, const ProbeJob &job) {
    std::vector<uint64_t> h(job.tiles + 1, 0);
    if (job.tiles) {
        XH_CHECK_HIP(hipMemcpyAsync(h.data(), job.toff.p, (job.tiles + 1) * sizeof(uint64_t), hipMemcpyDeviceToHost,
                                    ctx->stream));
        ctx->sync();
    }
    return h;
}

void probe_emit_range(Ctx *ctx, const ProbeJob &job, uint64_t t0, uint64_t t1, uint64_t rows, int out_arity,
                      const int oc[4], uint64_t *out0, uint64_t *out1) {
    if (t1 <= t0) return;
    ProbeArgs a = probe_args(job);
    OutSpec spec{out_arity, {oc[0], oc[1], oc[2], oc[3]}};
    const uint64_t tr = tile_rows(job.items);
    uint64_t nprobe = std::min<uint64_t>(job.n, t1 * tr) - t0 * tr;
    // per probe row: the row (8 B) and its run, as a 16-byte slot or as the count
    // pass's 12-byte record; per match: payload 4 B + output 8 B
    Prof prof(ctx, XLOG_HIP_KERNEL_PROBE_EMIT,
              (job.pre_cnt ? 20.0 : 24.0) * (double)nprobe + (4.0 + 8.0 * (out_arity > 2 ? 2 : 1)) * (double)rows);
    hipLaunchKernelGGL(k_probe_emit<JITEMS>, dim3((unsigned)(t1 - t0)), dim3(JB), 0, ctx->stream, a, job.toff.p, t0,
                       spec, out0, out1);
    XH_CHECK_HIP(hipGetLastError());
}

uint64_t join_probe_general(Ctx *ctx, const uint64_t *probe, uint64_t n, int pcol, const RunIndex &ix,
                            const uint32_t *payload, int out_arity, const int oc[4], uint64_t **out0,
                            uint64_t **out1) {
    *out0 = nullptr;
    if (out1) *out1 = nullptr;
    ProbeJob job;
    job.probe = probe;
    job.n = n;
    job.pcol = pcol;
    job.ix = &ix;
    job.payload = payload;
    uint64_t total = probe_prepare(ctx, job);
    if (total == 0) return 0;
    uint64_t *o0 = static_cast<uint64_t *>(ctx->alloc(total * sizeof(uint64_t)));
    uint64_t *o1 = (out_arity > 2) ? static_cast<uint64_t *>(ctx->alloc(total * sizeof(uint64_t))) : nullptr;
    probe_emit_range(ctx, job, 0, job.tiles, total, out_arity, oc, o0, o1);
    *out0 = o0;
    if (out1) *out1 = o1;
    return total;
}

uint64_t join_probe_project(Ctx *ctx, const uint64_t *probe, uint64_t n, int pcol, const RunIndex &ix,
                            const uint32_t *payload, int oc0, int oc1, uint64_t **out) {
    int oc[4] = {oc0, oc1, 0, 0};
    return join_probe_general(ctx, probe, n, pcol, ix, payload, 2, oc, out, nullptr);
}

void join_match_flags(Ctx *ctx, const uint64_t *probe, uint64_t n, int pcol, const RunIndex &ix, int want,
                      uint8_t *flags) {
    if (n == 0) return;
    ProbeArgs a{probe, n, pcol, ix.table.p, ix.table_mask, table_bits(ix), nullptr, nullptr, nullptr, nullptr,
                nullptr, nullptr, nullptr, nullptr};
    hipLaunchKernelGGL(k_match_flags, dim3(grid_for(n, 256, 16384)), dim3(256), 0, ctx->stream, a, want, flags);
    XH_CHECK_HIP(hipGetLastError());
}

void wcoj_triangle_flags(Ctx *ctx, const uint64_t *mask, uint64_t n, int mask_swap, const RunIndex &P,
                         const uint32_t *p_payload, const RunIndex &Q, const uint32_t *q_payload, uint8_t *flags) {
    if (n == 0) return;
    hipLaunchKernelGGL(k_wcoj_triangle, dim3(grid_for(n, 256, 16384)), dim3(256), 0, ctx->stream, mask, n, mask_swap,
                       P.table.p, P.table_mask, table_bits(P), p_payload, Q.table.p, Q.table_mask, table_bits(Q),
                       q_payload, flags);
    XH_CHECK_HIP(hipGetLastError());
}
void join_match2_flags(Ctx *ctx, const uint64_t *probe, uint64_t n, int pcol, const RunIndex &ix, const uint32_t *payload,
                       uint8_t *flags) {
    if (n == 0) return;
    ProbeArgs a{probe, n, pcol, ix.table.p, ix.table_mask, table_bits(ix), payload, nullptr, nullptr, nullptr,
                nullptr, nullptr, nullptr, nullptr};
    hipLaunchKernelGGL(k_match2_flags, dim3(grid_for(n, 256, 16384)), dim3(256), 0, ctx->stream, a, flags);
    XH_CHECK_HIP(hipGetLastError());
}

void smj_lookup(Ctx *ctx, const uint64_t *l, uint64_t nl, int pcol, const uint32_t *run_key, const uint64_t *run_start,
                uint64_t nr, uint64_t *start, uint32_t *cnt) {
    if (nl == 0) return;
    const uint64_t tiles = (nl + nr + SMJ_TILE - 1) / SMJ_TILE;
    XH_REQUIRE(tiles < (1ull << 31), XLOG_HIP_CAPACITY_OVERFLOW, "sort-merge join: input too large");
    Buf<uint64_t> split(ctx, tiles + 1);
    hipLaunchKernelGGL(k_smj_partition, dim3((unsigned)((tiles + 1 + 255) / 256)), dim3(256), 0, ctx->stream, l, nl, pcol,
                       run_key, nr, tiles, split.p);
    hipLaunchKernelGGL(k_smj_lookup, dim3((unsigned)tiles), dim3(SMJ_BLOCK), 0, ctx->stream, l, nl, pcol, run_key,
                       run_start, nr, split.p, start, cnt);
    XH_CHECK_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Order-preserving join + project: helpers for emitting the projected join
// already sorted by (left column, right payload).
// ---------------------------------------------------------------------------
namespace {

__device__ __forceinline__ uint32_t packed_col(uint64_t row, int arity, int c) {
    return arity == 1 ? (uint32_t)row : (c == 0 ? (uint32_t)(row >> 32) : (uint32_t)row);
}

__global__ void k_left_keys(const uint64_t *__restrict__ l, uint64_t n, int arity, int oc0, int jk,
                            uint64_t *__restrict__ out) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        uint64_t r = l[i];
        out[i] = ((uint64_t)packed_col(r, arity, oc0) << 32) | packed_col(r, arity, jk);
    }
}

// first row of every group of >= 2 consecutive rows with the same high word
__global__ void k_group_heads(const uint64_t *__restrict__ k, uint64_t n, uint8_t *__restrict__ flags) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        uint32_t h = (uint32_t)(k[i] >> 32);
        bool next_same = i + 1 < n && (uint32_t)(k[i + 1] >> 32) == h;
        bool prev_same = i > 0 && (uint32_t)(k[i - 1] >> 32) == h;
        flags[i] = next_same && !prev_same;
    }
}

// [start, end) of the run of high word hw in sorted out[0..n)
// seg[2i], seg[2i + 1] = start and length of head i's rows in out; *max_len
// (when given) = the largest length
__global__ void k_find_segments(const uint64_t *__restrict__ out, uint64_t n, const uint64_t *__restrict__ heads,
                                uint64_t nh, uint64_t *__restrict__ seg, unsigned long long *max_len,
                                const uint64_t *d_n) {
    if (d_n) n = *d_n;  // the data length on the device
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    unsigned long long mx = 0;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nh; i += stride) {
        uint32_t hw = (uint32_t)(heads[i] >> 32);
        uint64_t lo = 0, hi = n;
        while (lo < hi) {
            uint64_t m = (lo + hi) >> 1;
            if ((uint32_t)(out[m] >> 32) < hw) lo = m + 1; else hi = m;
        }
        uint64_t s = lo;
        hi = n;
        while (lo < hi) {
            uint64_t m = (lo + hi) >> 1;
            if ((uint32_t)(out[m] >> 32) <= hw) lo = m + 1; else hi = m;
        }
        seg[2 * i] = s;
        seg[2 * i + 1] = lo - s;
        mx = lo - s > mx ? lo - s : mx;
    }
    if (max_len) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const unsigned long long t = __shfl_xor(mx, o, WAVE);
            mx = t > mx ? t : mx;
        }
        if ((threadIdx.x & (WAVE - 1)) == 0 && mx) atomicMax(max_len, mx);
    }
}

constexpr int SEG_MAX = 4096;

// One wave per segment of 2..64 keys (segment w, or which[w] when a list is
// given; other lengths are left alone): bitonic sort across the lanes (one key
// per lane, padding keys sort last).
constexpr int SEGW_WAVES = 4;
__global__ __launch_bounds__(SEGW_WAVES * WAVE) void k_segsort_wave(uint64_t *__restrict__ data,
                                                                   const uint64_t *__restrict__ seg,
                                                                   const uint32_t *__restrict__ which, uint64_t nw) {
    const uint64_t w = (uint64_t)blockIdx.x * SEGW_WAVES + (threadIdx.x >> 6);
    if (w >= nw) return;
    const int lane = threadIdx.x & (WAVE - 1);
    const uint64_t q = which ? which[w] : w;
    const uint64_t start = seg[2 * q], len = seg[2 * q + 1];
    if (len < 2 || len > (uint64_t)WAVE) return;
    uint64_t x = (uint64_t)lane < len ? data[start + lane] : ~0ull;
#pragma unroll
    for (int k = 2; k <= WAVE; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const uint64_t y = ((uint64_t)(uint32_t)__shfl_xor((int)(uint32_t)(x >> 32), j, WAVE) << 32) |
                               (uint32_t)__shfl_xor((int)(uint32_t)x, j, WAVE);
            // the lower lane of the pair keeps the smaller key in an ascending
            // block (bit k of the lane clear), the larger one otherwise
            const bool lower = (lane & j) == 0, asc = (lane & k) == 0;
            const uint64_t lo = x < y ? x : y, hi = x < y ? y : x;
            x = (lower == asc) ? lo : hi;
        }
    }
    if ((uint64_t)lane < len) data[start + lane] = x;
}

// One block per segment of 65..SEG_MAX keys (segment blockIdx.x + first;
// other lengths are left alone): bitonic sort in LDS.
__global__ __launch_bounds__(256) void k_segsort(uint64_t *__restrict__ data, const uint64_t *__restrict__ seg,
                                                 uint64_t first) {
    __shared__ uint64_t s[SEG_MAX];
    const uint64_t q = first + blockIdx.x;
    const uint64_t start = seg[2 * q], len = seg[2 * q + 1];
    if (len <= (uint64_t)WAVE || len > (uint64_t)SEG_MAX) return;  // block-uniform
    uint32_t m = 1;
    while (m < len) m <<= 1;
    for (uint32_t i = threadIdx.x; i < m; i += blockDim.x) s[i] = i < len ? data[start + i] : ~0ull;
    __syncthreads();
    for (uint32_t k = 2; k <= m; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t i = threadIdx.x; i < m; i += blockDim.x) {
                uint32_t p = i ^ j;
                if (p > i) {
                    uint64_t a = s[i], b = s[p];
                    bool up = (i & k) == 0;
                    if ((a > b) == up) {
                        s[i] = b;
                        s[p] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    for (uint32_t i = threadIdx.x; i < len; i += blockDim.x) data[start + i] = s[i];
}

}  // namespace

void left_keys(Ctx *ctx, const uint64_t *l, uint64_t n, int arity, int oc0, int jk, uint64_t *out) {
    if (!n) return;
    hipLaunchKernelGGL(k_left_keys, dim3(grid_for(n, 256, 16384)), dim3(256), 0, ctx->stream, l, n, arity, oc0, jk,
                       out);
    XH_CHECK_HIP(hipGetLastError());
}

void group_head_flags(Ctx *ctx, const uint64_t *k, uint64_t n, uint8_t *flags) {
    if (!n) return;
    hipLaunchKernelGGL(k_group_heads, dim3(grid_for(n, 256, 16384)), dim3(256), 0, ctx->stream, k, n, flags);
    XH_CHECK_HIP(hipGetLastError());
}

__global__ void k_mark_members(const uint64_t *__restrict__ pos, uint64_t nm, int32_t *__restrict__ gsel,
                               const uint64_t *d_nm) {
    if (d_nm) nm = *d_nm;
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nm; i += stride) gsel[pos[i]] = -2;
}

// Row groups of probe keys sorted by their high word (the out column): rows
// that share it with a neighbour.  gsel[n] receives -1 for lone rows, -2 for
// group members and, at each group's first row, the group number; mkeys /
// mpos (n entries each) receive the members' keys and rows, hkeys / hpos (n
// entries each, hpos optional) the heads' keys and rows; the member count
// goes to *d_nm and the group count to *d_nh, on the device.
void group_rows_async(Ctx *ctx, const uint64_t *k, uint64_t n, int32_t *gsel, uint64_t *mkeys, uint64_t *mpos,
                      uint64_t *hkeys, uint64_t *hpos, uint64_t *d_nm, uint64_t *d_nh) {
    if (!n) {
        fill_u64(ctx, d_nm, 0ull, 1);
        fill_u64(ctx, d_nh, 0ull, 1);
        return;
    }
    fill_u32(ctx, reinterpret_cast<uint32_t *>(gsel), 0xFFFFFFFFu, n);
    select_group_members(ctx, k, n, mkeys, mpos, d_nm);
    hipLaunchKernelGGL(k_mark_members, dim3(grid_for(n, 256, (unsigned)ctx->num_cus * 4)), dim3(256), 0, ctx->stream,
                       mpos, n, gsel, d_nm);
    XH_CHECK_HIP(hipGetLastError());
    select_group_heads(ctx, mkeys, n, mpos, hkeys, gsel, d_nh, d_nm, hpos);
}
void group_segments(Ctx *ctx, const uint64_t *sorted, uint64_t n, const uint64_t *head_keys, uint64_t nh,
                    uint64_t *seg, const uint64_t *d_n) {
    if (!nh) return;
    hipLaunchKernelGGL(k_find_segments, dim3(grid_for(nh, 256, 16384)), dim3(256), 0, ctx->stream, sorted, n,
                       head_keys, nh, seg, nullptr, d_n);
    XH_CHECK_HIP(hipGetLastError());
}

// Sorts the runs of equal high word named by heads[0..nh) inside sorted-by-
// high-word data[0..n).  Runs of up to one wave are sorted in registers, up
// to SEG_MAX keys in LDS, longer ones by the radix sort on the slice.  The
// async part finds the runs (seg: 2 * nh entries) and sorts those of up to one
// wave, with the longest run's length in *d_max; sort_segments_long sorts the
// longer ones once the host knows that length.
void sort_segments_async(Ctx *ctx, uint64_t *data, uint64_t n, const uint64_t *heads, uint64_t nh, uint64_t *seg,
                         unsigned long long *d_max) {
    fill_u64(ctx, reinterpret_cast<uint64_t *>(d_max), 0ull, 1);
    if (!nh || !n) return;
    hipLaunchKernelGGL(k_find_segments, dim3(grid_for(nh, 256, 16384)), dim3(256), 0, ctx->stream, data, n, heads,
                       nh, seg, d_max, nullptr);
    XH_CHECK_HIP(hipGetLastError());
    // segments of up to 64 keys (the common case: probe rows sharing an out
    // column) need no host round trip: one wave per segment, all segments
    hipLaunchKernelGGL(k_segsort_wave, dim3((unsigned)((nh + SEGW_WAVES - 1) / SEGW_WAVES)), dim3(SEGW_WAVES * WAVE),
                       0, ctx->stream, data, seg, nullptr, nh);
    XH_CHECK_HIP(hipGetLastError());
}
void sort_segments_long(Ctx *ctx, uint64_t *data, const uint64_t *seg, uint64_t nh, uint64_t max_len) {
    if (max_len <= (uint64_t)WAVE) return;
    for (uint64_t off = 0; off < nh; off += (1u << 30)) {
        const uint64_t cnt = std::min<uint64_t>(nh - off, 1u << 30);
        hipLaunchKernelGGL(k_segsort, dim3((unsigned)cnt), dim3(256), 0, ctx->stream, data, seg, off);
        XH_CHECK_HIP(hipGetLastError());
    }
    if (max_len <= (uint64_t)SEG_MAX) return;
    // longer segments: radix sort of the slice (low words; the high words are
    // equal inside a segment)
    std::vector<uint64_t> h(2 * nh);
    XH_CHECK_HIP(hipMemcpyAsync(h.data(), seg, 2 * nh * sizeof(uint64_t), hipMemcpyDeviceToHost, ctx->stream));
    ctx->sync();
    for (uint64_t i = 0; i < nh; ++i) {
        const uint64_t st = h[2 * i], len = h[2 * i + 1];
        if (len <= (uint64_t)SEG_MAX) continue;
        uint64_t *a = data + st;
        uint64_t *b = static_cast<uint64_t *>(ctx->alloc(len * sizeof(uint64_t)));
        uint64_t *k0 = a, *k1 = b;
        uint32_t *v0 = nullptr, *v1 = nullptr;
        radix_sort_u64(ctx, &k0, &k1, &v0, &v1, len, 0, 4);
        if (k0 != a) XH_CHECK_HIP(hipMemcpyAsync(a, k0, len * 8, hipMemcpyDeviceToDevice, ctx->stream));
        ctx->free(b);
    }
}
}  // namespace xh

namespace xh {
namespace {

// Nested-loop inner join on one key column.  One wave per left row; the
// lanes stride the right rows 64 at a time and a ballot per step gives the
// matches, so every left row's outputs come in right-row order.  The count
// launch (emit == 0) writes per-left-row match counts; the emit launch reads
// their exclusive prefix and writes (left columns ++ right columns).
constexpr int NLJ_WAVES = 4;
__global__ __launch_bounds__(NLJ_WAVES * WAVE) void k_nlj(const uint64_t *__restrict__ l, uint64_t nl, int la, int lk,
                                                         const uint64_t *__restrict__ r, uint64_t nr, int ra, int rk,
                                                         uint64_t *__restrict__ cnt_off, int emit, OutSpec spec,
                                                         uint64_t *__restrict__ out0, uint64_t *__restrict__ out1) {
    const int lane = threadIdx.x & (WAVE - 1);
    const uint64_t row = (uint64_t)blockIdx.x * NLJ_WAVES + (threadIdx.x >> 6);
    if (row >= nl) return;
    const uint64_t lw = l[row];
    const uint32_t lc0 = packed_col(lw, la, 0), lc1 = la == 2 ? packed_col(lw, la, 1) : 0u;
    const uint32_t key = lk == 0 ? lc0 : lc1;
    const uint64_t lt_mask = (1ull << lane) - 1ull;
    uint64_t o = emit ? cnt_off[row] : 0ull;
    for (uint64_t b = 0; b < nr; b += WAVE) {
        const uint64_t j = b + (uint64_t)lane;
        uint32_t rc0 = 0, rc1 = 0;
        bool m = false;
        if (j < nr) {
            const uint64_t rw = r[j];
            rc0 = packed_col(rw, ra, 0);
            rc1 = ra == 2 ? packed_col(rw, ra, 1) : 0u;
            m = (rk == 0 ? rc0 : rc1) == key;
        }
        const uint64_t bal = __ballot(m);
        if (emit && m) {
            const uint64_t pos = o + (uint64_t)__popcll(bal & lt_mask);
            const uint32_t v[4] = {lc0, lc1, rc0, rc1};
            uint64_t w0, w1;
            make_words(spec, v, &w0, &w1);
            out0[pos] = w0;
            if (out1) out1[pos] = w1;
        }
        o += (uint64_t)__popcll(bal);
    }
    if (!emit && lane == 0) cnt_off[row] = o;
}

}  // namespace

uint64_t nested_loop_join(Ctx *ctx, const uint64_t *l, uint64_t nl, int la, int lk, const uint64_t *r, uint64_t nr,
                          int ra, int rk, uint64_t **out0, uint64_t **out1) {
    *out0 = *out1 = nullptr;
    if (nl == 0 || nr == 0) return 0;
    Buf<uint64_t> off(ctx, nl + 1);
    OutSpec spec{la + ra, {0, 1, 2, 3}};
    if (la == 1) {  // v = {l.c0, l.c1, r.c0, r.c1}: output = left columns ++ right columns
        spec.oc[1] = 2;
        spec.oc[2] = 3;
    }
    const unsigned grid = (unsigned)((nl + NLJ_WAVES - 1) / NLJ_WAVES);
    hipLaunchKernelGGL(k_nlj, dim3(grid), dim3(NLJ_WAVES * WAVE), 0, ctx->stream, l, nl, la, lk, r, nr, ra, rk, off.p,
                       0, spec, nullptr, nullptr);
    XH_CHECK_HIP(hipGetLastError());
    scan_u64_inplace(ctx, off.p, nl, off.p + nl);
    ctx->read_scalars(off.p + nl, 1);
    const uint64_t total = ctx->host_scalars[0];
    if (total == 0) return 0;
    *out0 = static_cast<uint64_t *>(ctx->alloc(total * sizeof(uint64_t)));
    if (spec.arity > 2) *out1 = static_cast<uint64_t *>(ctx->alloc(total * sizeof(uint64_t)));
    hipLaunchKernelGGL(k_nlj, dim3(grid), dim3(NLJ_WAVES * WAVE), 0, ctx->stream, l, nl, la, lk, r, nr, ra, rk, off.p,
                       1, spec, *out0, *out1);
    XH_CHECK_HIP(hipGetLastError());
    return total;
}

}  // namespace xh
