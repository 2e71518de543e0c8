// Dense-domain semi-naive fixpoint for programs whose rules are chains of
// binary relations, for gfx950.
//
// The reference evaluates every recursive rule with the join route
// (Executor::execute_recursive_scc, crates/xlog-runtime/src/executor/
// recursive.rs:447-957) and keeps a dense factorized delta only for the
// transitive-closure shape (fj_delta_novel_u32_recorded, crates/xlog-cuda/src/
// provider/fj_delta.rs:117-490).  Here any rule
//     head(v0, vk) :- a1(v0, v1), a2(v1, v2), ..., ak(v_{k-1}, vk)
// (atoms in any order, each read forward or with its columns swapped) is a
// chain of boolean products over the id domain, so a whole program of such
// rules (transitive closure, Andersen points-to, same-generation ...) runs
// with every relation as a domain x domain bit matrix resident in HBM:
//
//   IDB predicate  : R (full), D (delta), C (candidates), and R^T / D^T when
//                    some rule reads it backward; each with a row mask (bit x
//                    set iff row x is non-empty) so empty rows are skipped.
//   EDB predicate  : CSR (row_ptr, adj), forward and / or transposed.
//
// One product  out[x] = OR_{y in left[x], right[y] != 0} right[y]  is one
// launch of k_chain_product (a block per row x).  A chain of k atoms is k-1
// products evaluated left to right into two ping-pong temporaries; the last
// product ORs into the head's candidate matrix.  Per iteration, for every
// rule and every IDB occurrence whose delta is non-empty, the chain runs with
// the delta at that occurrence and the full relation elsewhere -- the same
// variants as the join route, IDB atoms before the delta reading R minus D
// (P) -- then k_chain_finalize per IDB predicate does
//   P |= D;  D = C & ~R;  R |= D;  C = 0
// and, for predicates read backward, k_transpose_delta rebuilds D^T and
// updates R^T and P^T from 64 x 64 bit tiles of the changed row blocks.
// and counts |D|; the counts are the only values read back.  Results leave
// the device once, at convergence, as canonical rows (bitmap_emit).
#include "internal.hpp"

namespace xh {

namespace {

constexpr int PTB = 512;           // product block: 8 waves
constexpr int PNW = PTB / WAVE;
constexpr int LCHUNK_WORDS = 64;   // left-row bitmap words compacted per round (<= 4096 ids)
constexpr int FTB = 256;           // row-op block
#ifndef XH_GATHER_UNROLL
#define XH_GATHER_UNROLL 8
#endif
constexpr int GATHER_UNROLL = XH_GATHER_UNROLL;  // right-row loads in flight per wave
constexpr uint32_t MAX_DOMAIN = 1u << 17;
// Device counters that many blocks add to are spread over SPREAD addresses
// (block id mod SPREAD), summed when read back: one address would serialise
// tens of thousands of atomics per launch in L2.
constexpr int SPREAD = Ctx::PROF_WORK_SPREAD;

// One operand of a product: a bitmap (bits != null) or a CSR (row_ptr, adj);
// mask bit x is set iff row x is non-empty (exact for CSR and for R / D / C /
// R^T / D^T; for product temporaries rows without their bit hold garbage and
// are never read).
struct Operand {
    const uint64_t *bits;
    const uint64_t *row_ptr;
    const uint32_t *adj;
    const uint64_t *mask;
};

__device__ __forceinline__ bool bit_of(const uint64_t *m, uint32_t x) { return (m[x >> 6] >> (x & 63)) & 1ull; }

__device__ __forceinline__ void set_bit(uint64_t *m, uint32_t x) {
    const uint64_t b = 1ull << (x & 63);
    // a stale read only costs a redundant atomic
    if (!(m[x >> 6] & b)) atomicOr((unsigned long long *)&m[x >> 6], (unsigned long long)b);
}

// out[x] (= or |=) OR over the left row's ids y whose right row is non-empty
// of right[y].  Left CSR rows are consumed PTB entries per round, left bitmap
// rows LCHUNK_WORDS words per round; each round's ids are compacted into
// s_y.  A bitmap right row is read in 64-word stripes, one coalesced 512-byte
// load per id per stripe (a lane per word), by waves that split the stripes
// and, when there are fewer stripes than waves, the ids; a CSR right row is
// expanded by threads over ids with LDS atomics.  The row accumulates in LDS.
template <bool LCSR, bool RCSR, bool ACC>
__global__ __launch_bounds__(PTB) void k_chain_product(uint32_t words, Operand L, Operand R, uint64_t *__restrict__ O,
                                                       uint64_t *__restrict__ omask,
                                                       unsigned long long *__restrict__ work) {
    extern __shared__ uint64_t s_acc[];  // words
    __shared__ uint32_t s_y[LCHUNK_WORDS * 64];
    __shared__ uint64_t s_bits[LCHUNK_WORDS];
    __shared__ uint32_t s_woff[LCHUNK_WORDS + 1];
    __shared__ uint32_t s_any;
    __shared__ unsigned long long s_moved;
    const uint32_t x = blockIdx.x;
    if (!bit_of(L.mask, x)) return;  // block-uniform
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    for (uint32_t w = tid; w < words; w += PTB) s_acc[w] = 0ull;
    if (tid == 0) {
        s_any = 0u;
        s_moved = 0ull;
    }
    __syncthreads();
    uint64_t lbeg = 0, lend = words;
    if (LCSR) {
        lbeg = L.row_ptr[x];
        lend = L.row_ptr[x + 1];
    }
    const uint64_t step = LCSR ? (uint64_t)PTB : (uint64_t)LCHUNK_WORDS;
    const uint64_t lt_mask = (1ull << lane) - 1ull;
    const uint32_t ns = (words + 63) / 64;
    // bytes this block reads and writes (left row, gathered right rows, output row), for profiling
    uint64_t moved = (LCSR ? 4ull * (lend - lbeg) : 8ull * words) + 8ull * words, adj_bytes = 0;
    for (uint64_t c0 = lbeg; c0 < lend; c0 += step) {
        if (LCSR) {
            const uint64_t e = c0 + tid;
            const uint32_t y = e < lend ? L.adj[e] : 0u;
            const bool keep = e < lend && bit_of(R.mask, y);
            const uint64_t bal = __ballot(keep);
            if (lane == 0) s_woff[wave] = (uint32_t)__popcll(bal);
            __syncthreads();
            if (tid == 0) {
                uint32_t run = 0;
                for (int q = 0; q < PNW; ++q) {
                    const uint32_t c = s_woff[q];
                    s_woff[q] = run;
                    run += c;
                }
                s_woff[LCHUNK_WORDS] = run;
            }
            __syncthreads();
            if (keep) s_y[s_woff[wave] + (uint32_t)__popcll(bal & lt_mask)] = y;
        } else {
            if (wave == 0) {
                const uint64_t w = c0 + lane;
                const uint64_t bits = w < words ? L.bits[(uint64_t)x * words + w] & R.mask[w] : 0ull;
                const uint32_t pc = (uint32_t)__popcll(bits);
                uint32_t incl = pc;
#pragma unroll
                for (int o = 1; o < WAVE; o <<= 1) {
                    const uint32_t t = __shfl_up(incl, o, WAVE);
                    if (lane >= o) incl += t;
                }
                s_bits[lane] = bits;
                s_woff[lane] = incl - pc;
                if (lane == WAVE - 1) s_woff[LCHUNK_WORDS] = incl;
            }
            __syncthreads();
            if (s_woff[LCHUNK_WORDS])
                for (int j = wave; j < LCHUNK_WORDS; j += PNW) {
                    const uint64_t bits = s_bits[j];
                    if ((bits >> lane) & 1ull)
                        s_y[s_woff[j] + (uint32_t)__popcll(bits & lt_mask)] = (uint32_t)((c0 + j) * 64 + lane);
                }
        }
        __syncthreads();
        const uint32_t T = s_woff[LCHUNK_WORDS];
        if (T) {
            if (RCSR) {
                moved += 16ull * T;
                for (uint32_t q = tid; q < T; q += PTB) {
                    const uint32_t y = s_y[q];
                    const uint64_t b = R.row_ptr[y], f = R.row_ptr[y + 1];
                    adj_bytes += 4ull * (f - b);
                    for (uint64_t e = b; e < f; ++e) {
                        const uint32_t z = R.adj[e];
                        atomicOr((unsigned long long *)&s_acc[z >> 6], 1ull << (z & 63));
                    }
                }
            } else {
                moved += 8ull * words * T;
                // The round's (stripe, id) pairs, stripe-major, split into equal
                // contiguous ranges, one per wave: a wave ORs each run of ids
                // of one stripe in registers (GATHER_UNROLL row loads in
                // flight, a lane per word) and folds the run into LDS.
                const uint32_t N = ns * T, per = (N + PNW - 1) / PNW;
                uint32_t i = wave * per;
                const uint32_t iend = min(N, i + per);
                while (i < iend) {
                    const uint32_t s = i / T, j0 = i - s * T;
                    const uint32_t j1 = min(T, j0 + (iend - i));
                    const uint32_t w = s * 64 + lane;
                    if (w < words) {
                        const uint64_t *col = R.bits + w;
                        uint64_t acc = 0ull;
                        uint32_t j = j0;
                        for (; j + GATHER_UNROLL <= j1; j += GATHER_UNROLL) {
                            uint64_t v[GATHER_UNROLL];
#pragma unroll
                            for (int u = 0; u < GATHER_UNROLL; ++u) v[u] = col[(uint64_t)s_y[j + u] * words];
#pragma unroll
                            for (int u = 0; u < GATHER_UNROLL; ++u) acc |= v[u];
                        }
                        for (; j < j1; ++j) acc |= col[(uint64_t)s_y[j] * words];
                        if (acc) atomicOr((unsigned long long *)&s_acc[w], acc);
                    }
                    i += j1 - j0;
                }
            }
        }
        __syncthreads();
    }
    uint64_t *orow = O + (uint64_t)x * words;
    bool any = false;
    for (uint32_t w = tid; w < words; w += PTB) {
        const uint64_t a = s_acc[w];
        if (ACC) {
            if (a) orow[w] |= a;
        } else {
            orow[w] = a;
        }
        any |= a != 0ull;
    }
    if (__ballot(any) != 0ull && lane == 0) s_any = 1u;
    if (RCSR && work && adj_bytes) atomicAdd(&s_moved, (unsigned long long)adj_bytes);
    __syncthreads();
    if (tid == 0) {
        if (s_any) set_bit(omask, x);
        if (work) atomicAdd(&work[blockIdx.x & (SPREAD - 1)], (unsigned long long)moved + s_moved);
    }
}

// Output of a fused product: the new delta is written straight into the
// candidate matrix, R is updated and the delta counted, so no separate
// finalize pass touches the row again.  With full_rows every row the product
// reaches is written whole (zero words included), so the matrix needs no
// clearing beforehand: its other rows keep stale bits under a clear mask bit.
// `zero` (when set) is a row mask of zero_words words that the launch clears
// on the side: the next iteration's delta mask, read by nothing in this one.
struct FusedArgs {
    uint64_t *R, *rmask;
    unsigned long long *count;
    uint32_t full_rows;
    uint64_t *zero;
    uint32_t zero_words;
};

constexpr int GW = 4;           // k_csr_gather: waves per block
constexpr int GWORDS = 8;       // words per lane per stripe group (a group = 512 words)
#ifndef XH_GATHER_NR
#define XH_GATHER_NR 2
#endif
#ifndef XH_GATHER_WAVES
#define XH_GATHER_WAVES 8192
#endif
constexpr int GNR = XH_GATHER_NR;  // right rows gathered per round (GNR x GWORDS loads in flight per lane)
constexpr uint32_t GATHER_WAVES = XH_GATHER_WAVES;  // waves per launch the row batches aim at
constexpr uint32_t GATHER_MAX_BATCH = 32;            // rows per wave batch (a power of two <= 32)

enum { OUT_ASSIGN = 0, OUT_OR = 1, OUT_FUSED = 2 };

// rows per wave of the row-batched kernels: a power of two (so a batch never
// straddles a row-mask word) large enough to keep the launch near GATHER_WAVES waves
inline uint32_t row_batch(uint32_t domain) {
    uint32_t batch = 1;
    while (batch < GATHER_MAX_BATCH && (uint64_t)domain > (uint64_t)GATHER_WAVES * batch) batch *= 2;
    return batch;
}

// atomically m |= bits << x, bits covering rows x .. x + 63 (two words at most)
__device__ __forceinline__ void or_bits(uint64_t *m, uint32_t x, uint64_t bits) {
    const uint32_t sh = x & 63;
    if (bits << sh) atomicOr((unsigned long long *)&m[x >> 6], (unsigned long long)(bits << sh));
    if (sh && (bits >> (64 - sh))) atomicOr((unsigned long long *)&m[(x >> 6) + 1], (unsigned long long)(bits >> (64 - sh)));
}

// The fused last product of a variant with a CSR left operand (short rows:
// EDB relations) and a bitmap right operand.  A wave owns `batch` consecutive
// output rows: their row offsets come in one load (a lane per row), their
// adjacency and the right operand's row-mask bits 64 edges at a time (a lane
// per edge), so the dependent loads before any gather are paid once per batch,
// not per row.  Per row x, the ids y of x's edges whose right row is non-empty
// come from a ballot over the loaded edges; R[x] and the right rows are then
// loaded in one round (8 coalesced loads per lane per row: words
// g0 + lane + 64k of a 512-word stripe group; GNR right rows at a time) and
// new = acc & ~R[x], R[x] |= new, O[x] = new (O is the candidate matrix
// becoming the next delta: all zero, or written whole when fz.full_rows),
// counted.  A row with no such id is left alone.
// The rows that received bits are OR-ed into the output and R row masks once
// per batch, and the counts once per block.
// (For the non-fused products of short left rows the block-per-row
// k_chain_product measured faster: 4.3 against 6.8 ms per C5 fixpoint.)
__global__ __launch_bounds__(GW * WAVE) void k_csr_gather_fused(uint32_t domain, uint32_t words, uint32_t batch,
                                                          Operand L, Operand Rt, uint64_t *__restrict__ O,
                                                          uint64_t *__restrict__ omask, FusedArgs fz,
                                                          unsigned long long *__restrict__ work) {
    __shared__ unsigned long long s_cnt[GW], s_work[GW];
    const int lane = threadIdx.x & (WAVE - 1);
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    unsigned long long cnt = 0, moved = 0;  // per lane
    if (fz.zero)
        for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < fz.zero_words; i += gridDim.x * blockDim.x)
            fz.zero[i] = 0ull;
    const uint64_t x0 = ((uint64_t)blockIdx.x * GW + wave) * batch;
    if (x0 < domain) {
        const uint32_t nr = (uint32_t)(domain - x0 < batch ? domain - x0 : batch);
        const uint64_t rp = (uint32_t)lane <= nr ? L.row_ptr[x0 + lane] : 0ull;
        const uint64_t ebeg = __shfl(rp, 0, WAVE), eend = __shfl(rp, (int)nr, WAVE);
        if (lane == 0) moved += 4ull * (eend - ebeg);
        // the loaded edge chunk: edges c0 + lane, their ids and whether their right row is non-empty
        uint64_t c0 = ebeg;
        uint32_t y = 0;
        bool keep = false;
        {
            const uint64_t e = c0 + lane;
            y = e < eend ? L.adj[e] : 0u;
            keep = e < eend && bit_of(Rt.mask, y);
        }
        uint64_t rows_set = 0;  // bit r: row x0 + r received new bits
        for (uint32_t r = 0; r < nr; ++r) {
            const uint64_t rb = __shfl(rp, (int)r, WAVE), re = __shfl(rp, (int)r + 1, WAVE);
            if (rb == re) continue;  // wave-uniform
            const uint64_t x = x0 + r;
            uint64_t *orow = O + x * words;
            uint64_t *rrow = fz.R + x * words;
            bool any = false;
            for (uint32_t g0 = 0; g0 < words; g0 += GWORDS * WAVE) {
                uint64_t acc[GWORDS], rv[GWORDS];
#pragma unroll
                for (int k = 0; k < GWORDS; ++k) acc[k] = rv[k] = 0ull;
                bool have_r = false;
                unsigned long long gathered = 0;
                for (uint64_t pos = rb; pos < re;) {  // wave-uniform walk over the row's edges
                    if (pos < c0 || pos >= c0 + WAVE) {
                        c0 = pos;
                        const uint64_t e = c0 + lane;
                        y = e < eend ? L.adj[e] : 0u;
                        keep = e < eend && bit_of(Rt.mask, y);
                    }
                    const uint64_t lim = re < c0 + WAVE ? re : c0 + WAVE;
                    const uint64_t e = c0 + lane;
                    uint64_t bal = __ballot(keep && e >= pos && e < lim);
                    pos = lim;
                    if (!bal) continue;
                    gathered += (unsigned long long)__popcll(bal);
                    if (!have_r) {  // R[x]'s group, loaded with the first right rows
                        have_r = true;
#pragma unroll
                        for (int k = 0; k < GWORDS; ++k) {
                            const uint32_t w = g0 + lane + 64u * k;
                            rv[k] = w < words ? rrow[w] : 0ull;
                        }
                    }
                    while (bal) {  // GNR right rows at a time
                        uint32_t ys[GNR];
                        bool ok[GNR];
#pragma unroll
                        for (int j = 0; j < GNR; ++j) {
                            ok[j] = bal != 0ull;
                            const int s = ok[j] ? __builtin_ctzll(bal) : 0;
                            bal &= bal - 1ull;
                            ys[j] = (uint32_t)__shfl((int)y, s, WAVE);
                        }
                        uint64_t v[GNR][GWORDS];
#pragma unroll
                        for (int j = 0; j < GNR; ++j) {
                            const uint64_t *src = Rt.bits + (uint64_t)ys[j] * words + g0 + lane;
#pragma unroll
                            for (int k = 0; k < GWORDS; ++k)
                                v[j][k] = (ok[j] && g0 + lane + 64u * k < words) ? src[64 * k] : 0ull;
                        }
#pragma unroll
                        for (int j = 0; j < GNR; ++j)
#pragma unroll
                            for (int k = 0; k < GWORDS; ++k) acc[k] |= v[j][k];
                    }
                }
                if (!have_r) continue;  // no id of this row has a non-empty right row
                const uint32_t gw = words - g0 < GWORDS * WAVE ? words - g0 : GWORDS * WAVE;
                if (lane == 0) moved += 8ull * gw * (gathered + 1);  // the right rows and R[x]
#pragma unroll
                for (int k = 0; k < GWORDS; ++k) {
                    const uint32_t w = g0 + lane + 64u * k;
                    const uint64_t nw = acc[k] & ~rv[k];
                    if (w < words && nw) {
                        rrow[w] = rv[k] | nw;
                        orow[w] = nw;
                        cnt += (unsigned long long)__popcll(nw);
                        moved += 16ull;  // the R and O words written
                        any = true;
                    } else if (w < words && fz.full_rows) {
                        orow[w] = 0ull;
                        moved += 8ull;
                    }
                }
            }
            if (__ballot(any) != 0ull) rows_set |= 1ull << r;
        }
        if (lane == 0 && rows_set) {
            or_bits(omask, (uint32_t)x0, rows_set);
            or_bits(fz.rmask, (uint32_t)x0, rows_set);
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        cnt += __shfl_xor(cnt, o, WAVE);
        moved += __shfl_xor(moved, o, WAVE);
    }
    if (lane == 0) {
        s_cnt[wave] = cnt;
        s_work[wave] = moved;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long c = 0, m = 0;
#pragma unroll
        for (int i = 0; i < GW; ++i) {
            c += s_cnt[i];
            m += s_work[i];
        }
        if (c) atomicAdd(&fz.count[blockIdx.x & (SPREAD - 1)], c);
        if (work && m) atomicAdd(&work[blockIdx.x & (SPREAD - 1)], m);
    }
}

// zero the rows of B whose mask bit is set
__global__ __launch_bounds__(FTB) void k_clear_rows(uint32_t words, uint64_t *__restrict__ B,
                                                    const uint64_t *__restrict__ mask) {
    const uint32_t x = blockIdx.x;
    if (!bit_of(mask, x)) return;
    for (uint32_t w = threadIdx.x; w < words; w += FTB) B[(uint64_t)x * words + w] = 0ull;
}

// totals[i] = sum of the SPREAD partial counts of entry i (iterations x predicates)
__global__ void k_sum_counts(const unsigned long long *__restrict__ parts, uint32_t n,
                             unsigned long long *__restrict__ totals) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    unsigned long long t = 0;
    for (int q = 0; q < SPREAD; ++q) t += parts[(uint64_t)i * SPREAD + q];
    totals[i] = t;
}

// C[x] |= B[x] for the rows of B's mask (a one-atom chain over an IDB operand)
__global__ __launch_bounds__(FTB) void k_or_rows(uint32_t words, const uint64_t *__restrict__ B,
                                                 const uint64_t *__restrict__ bmask, uint64_t *__restrict__ C,
                                                 uint64_t *__restrict__ cmask) {
    __shared__ uint32_t s_any;
    const uint32_t x = blockIdx.x;
    if (!bit_of(bmask, x)) return;
    if (threadIdx.x == 0) s_any = 0u;
    __syncthreads();
    bool any = false;
    for (uint32_t w = threadIdx.x; w < words; w += FTB) {
        const uint64_t b = B[(uint64_t)x * words + w];
        if (b) {
            C[(uint64_t)x * words + w] |= b;
            any = true;
        }
    }
    if (__ballot(any) != 0ull && (threadIdx.x & 63) == 0) s_any = 1u;
    __syncthreads();
    if (threadIdx.x == 0 && s_any) set_bit(cmask, x);
}

// bit (x, z) of B for every packed row (x the high word when x_hi, else the low)
__global__ void k_pairs_bits_mask(const uint64_t *__restrict__ rows, uint64_t n, int x_hi, uint32_t words,
                                  uint64_t *__restrict__ B, uint64_t *__restrict__ mask) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t e = rows[i];
        const uint32_t x = x_hi ? (uint32_t)(e >> 32) : (uint32_t)e;
        const uint32_t z = x_hi ? (uint32_t)e : (uint32_t)(e >> 32);
        atomicOr((unsigned long long *)&B[(uint64_t)x * words + (z >> 6)], 1ull << (z & 63));
        set_bit(mask, x);
    }
}

// Seed of a closure whose one exit rule copies an EDB relation E (read
// forward) into a head that starts empty: R = D = E as whole bit rows, one
// block per row, the row built in LDS from its CSR adjacency.  Writing every
// row whole replaces the zero-fills of R and D, and the seed needs neither the
// candidate matrix nor a finalize pass.
__global__ __launch_bounds__(FTB) void k_seed_rows(uint32_t words, const uint64_t *__restrict__ row_ptr,
                                                   const uint32_t *__restrict__ adj, uint64_t *__restrict__ R,
                                                   uint64_t *__restrict__ D) {
    extern __shared__ unsigned long long s_row[];  // `words` words
    const uint32_t x = blockIdx.x;
    for (uint32_t w = threadIdx.x; w < words; w += FTB) s_row[w] = 0ull;
    __syncthreads();
    const uint64_t b = row_ptr[x], e = row_ptr[x + 1];
    for (uint64_t i = b + threadIdx.x; i < e; i += FTB) {
        const uint32_t z = adj[i];
        atomicOr(&s_row[z >> 6], 1ull << (z & 63));
    }
    __syncthreads();
    for (uint32_t w = threadIdx.x; w < words; w += FTB) {
        const uint64_t v = s_row[w];
        R[(uint64_t)x * words + w] = v;
        D[(uint64_t)x * words + w] = v;
    }
}

// mask of the non-empty CSR rows, one mask word per thread
__global__ void k_csr_mask(const uint64_t *__restrict__ row_ptr, uint32_t nv, uint32_t words,
                           uint64_t *__restrict__ mask) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t w = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; w < words; w += stride) {
        uint64_t m = 0ull;
        for (uint32_t b = 0; b < 64; ++b) {
            const uint64_t v = w * 64 + b;
            if (v < nv && row_ptr[v + 1] > row_ptr[v]) m |= 1ull << b;
        }
        mask[w] = m;
    }
}

struct FinalizeArgs {
    uint64_t *C;
    const uint64_t *cmask;
    uint64_t *R, *rmask;
    uint64_t *D;
    const uint64_t *dmask_old;
    uint64_t *dmask_new;
    uint64_t *P, *pmask;  // R minus D (null when no rule reads it forward)
    unsigned long long *count;
    unsigned long long *work;  // profiling (or null): bytes of the row words loaded and stored
};

// Per row x with candidates or an old delta row:
//   P[x] |= D[x];  D[x] = C[x] & ~R[x];  R[x] |= D[x];  C[x] = 0
// (so that afterwards P = R minus the new D), sets the new delta / full
// row-mask bits and adds |D[x]| to the count.  A wave owns `batch` rows (a
// power of two, so their mask bits share one word, read once): per active
// row, C, the old D and P words come in one round of loads (8 per lane per
// 512-word group), R under the non-zero C words in a second, then the stores.
// Row-mask bits are OR-ed once per batch, the count once per block.
template <bool PREV>
__global__ __launch_bounds__(GW * WAVE) void k_chain_finalize(uint32_t domain, uint32_t words, uint32_t batch,
                                                              FinalizeArgs a) {
    __shared__ unsigned long long s_cnt[GW], s_work[GW];
    const int lane = threadIdx.x & (WAVE - 1);
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    unsigned long long cnt = 0;   // per lane
    unsigned long long moved = 0;  // per lane: words loaded or stored (counted when profiling)
    const uint32_t x0 = (blockIdx.x * GW + wave) * batch;
    if (x0 < domain) {
        const uint32_t nr = domain - x0 < batch ? domain - x0 : batch;
        const uint64_t rows = nr == 64 ? ~0ull : (1ull << nr) - 1ull;
        const uint64_t cm = (a.cmask[x0 >> 6] >> (x0 & 63)) & rows, dm = (a.dmask_old[x0 >> 6] >> (x0 & 63)) & rows;
        uint64_t active = cm | dm, dset = 0;
        while (active) {  // wave-uniform
            const int r = __builtin_ctzll(active);
            active &= active - 1ull;
            const bool c_on = (cm >> r) & 1ull, d_on = (dm >> r) & 1ull;
            const uint64_t base = (uint64_t)(x0 + r) * words;
            uint64_t *crow = a.C + base, *rrow = a.R + base, *drow = a.D + base;
            bool any = false;
            for (uint32_t g0 = 0; g0 < words; g0 += GWORDS * WAVE) {
                uint64_t cv[GWORDS], dv[GWORDS], pv[GWORDS], rv[GWORDS];
#pragma unroll
                for (int k = 0; k < GWORDS; ++k) {
                    const uint32_t w = g0 + lane + 64u * k;
                    const bool in = w < words;
                    cv[k] = in && c_on ? crow[w] : 0ull;
                    dv[k] = PREV && in && d_on ? drow[w] : 0ull;
                    pv[k] = PREV && in && d_on ? a.P[base + w] : 0ull;
                }
#pragma unroll
                for (int k = 0; k < GWORDS; ++k) {
                    const uint32_t w = g0 + lane + 64u * k;
                    rv[k] = cv[k] ? rrow[w] : 0ull;
                }
#pragma unroll
                for (int k = 0; k < GWORDS; ++k) {
                    const uint32_t w = g0 + lane + 64u * k;
                    if (w >= words) continue;
                    const uint64_t nw = cv[k] & ~rv[k];
                    // C, and D and P of an old delta row, are read; R under a non-zero C word
                    moved += (c_on ? 1u : 0u) + (PREV && d_on ? 2u : 0u) + (cv[k] ? 1u : 0u);
                    if (cv[k]) {
                        if (nw) rrow[w] = rv[k] | nw;
                        crow[w] = 0ull;
                        moved += nw ? 2u : 1u;
                    }
                    if (PREV && dv[k] && (pv[k] | dv[k]) != pv[k]) {
                        a.P[base + w] = pv[k] | dv[k];
                        ++moved;
                    }
                    if (d_on || nw) {
                        drow[w] = nw;
                        ++moved;
                    }
                    cnt += (unsigned long long)__popcll(nw);
                    any |= nw != 0ull;
                }
            }
            if (__ballot(any) != 0ull) dset |= 1ull << r;
        }
        if (lane == 0) {
            if (dset) {
                or_bits(a.dmask_new, x0, dset);
                or_bits(a.rmask, x0, dset);
            }
            if (PREV && dm) or_bits(a.pmask, x0, dm);  // the old delta rows were non-empty
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        cnt += __shfl_xor(cnt, o, WAVE);
        moved += __shfl_xor(moved, o, WAVE);
    }
    if (lane == 0) {
        s_cnt[wave] = cnt;
        s_work[wave] = moved;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long c = 0, m = 0;
#pragma unroll
        for (int i = 0; i < GW; ++i) {
            c += s_cnt[i];
            m += s_work[i];
        }
        if (c) atomicAdd(&a.count[blockIdx.x & (SPREAD - 1)], c);
        if (a.work && m) atomicAdd(&a.work[blockIdx.x & (SPREAD - 1)], 8ull * m);
    }
}

// 64 x 64 bit transpose across a wave: lane l holds row l on entry (bit c =
// column c) and column l on exit (bit r = row r).  Step s swaps the s x s
// off-diagonal blocks of every 2s x 2s block.
__device__ __forceinline__ uint64_t wave_transpose64(uint64_t w, int lane) {
    const uint64_t m[6] = {0x00000000FFFFFFFFull, 0x0000FFFF0000FFFFull, 0x00FF00FF00FF00FFull,
                           0x0F0F0F0F0F0F0F0Full, 0x3333333333333333ull, 0x5555555555555555ull};
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        const int s = 32 >> k;
        const uint64_t p = __shfl_xor(w, s, WAVE);
        w = (lane & s) ? ((w & ~m[k]) | ((p & ~m[k]) >> s)) : ((w & m[k]) | ((p & m[k]) << s));
    }
    return w;
}

constexpr int TT_WAVES = 4;  // transpose block: one 64-row block of D per wave
constexpr int TT_COLS = 8;   // word columns per wave (64-byte runs per lane, merged rows on the write side)

// Transposes after a finalize, for every 64-row block I of D where the old
// or the new delta has rows (elsewhere nothing changed): per word column J,
//   D^T[z][I] = column z of D's (I, J) tile;  P^T[z][I] = R^T[z][I] (R minus
//   the new D, transposed);  R^T[z][I] |= D^T[z][I].
// D^T's row mask is rebuilt (zeroed by the caller); R^T's and P^T's only
// grow, as R does.
__global__ __launch_bounds__(TT_WAVES * WAVE) void k_transpose_delta(
    uint32_t domain, uint32_t words, const uint64_t *__restrict__ D, const uint64_t *__restrict__ dmask_old,
    const uint64_t *__restrict__ dmask_new, uint64_t *__restrict__ DT, uint64_t *__restrict__ dtmask,
    uint64_t *__restrict__ RT, uint64_t *__restrict__ rtmask, uint64_t *__restrict__ PT,
    uint64_t *__restrict__ ptmask, unsigned long long *work) {
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const uint32_t I = blockIdx.y * TT_WAVES + wave;
    if (I >= words) return;                              // wave-uniform
    if ((dmask_old[I] | dmask_new[I]) == 0ull) return;  // wave-uniform
    const uint32_t J0 = blockIdx.x * TT_COLS;
    // profiling: D read, D^T written, R^T read and written (and P^T written) for the 64 x TT_COLS tile
    if (work && lane == 0 && J0 < words) {
        const uint32_t cols = words - J0 < (uint32_t)TT_COLS ? words - J0 : (uint32_t)TT_COLS;
        atomicAdd(&work[(blockIdx.x + blockIdx.y) & (SPREAD - 1)],
                  (unsigned long long)cols * 64ull * 8ull * (PT ? 5ull : 4ull));
    }
    const uint32_t row = I * 64 + lane;
    uint64_t v[TT_COLS];
#pragma unroll
    for (int j = 0; j < TT_COLS; ++j)
        v[j] = (row < domain && J0 + j < words) ? D[(uint64_t)row * words + J0 + j] : 0ull;
#pragma unroll
    for (int j = 0; j < TT_COLS; ++j) {
        const uint32_t J = J0 + j;
        if (J >= words) break;  // wave-uniform
        const uint64_t t = wave_transpose64(v[j], lane);
        const uint32_t z = J * 64 + lane;
        bool nd = false, np = false, nr = false;
        if (z < domain) {
            const uint64_t off = (uint64_t)z * words + I;
            const uint64_t r = RT[off];
            DT[off] = t;
            if (PT) PT[off] = r;
            if (t) RT[off] = r | t;
            nd = t != 0ull;
            np = r != 0ull;
            nr = (r | t) != 0ull;
        }
        const uint64_t bd = __ballot(nd), bp = __ballot(np), br = __ballot(nr);
        if (lane == 0) {
            if (bd) atomicOr((unsigned long long *)&dtmask[J], (unsigned long long)bd);
            if (PT && bp && (ptmask[J] & bp) != bp) atomicOr((unsigned long long *)&ptmask[J], (unsigned long long)bp);
            if (br && (rtmask[J] & br) != br) atomicOr((unsigned long long *)&rtmask[J], (unsigned long long)br);
        }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct BitRel {  // an IDB predicate
    Buf<uint64_t> R, D, C, RT, DT, P, PT;
    Buf<uint64_t> rmask, dmask[2], cmask, rtmask, dtmask, pmask, ptmask;
    int dcur = 0;
    // when every iteration is fused: a third delta mask, cleared by the fused
    // product while the other two are read and written (spare_zeroed: it was)
    Buf<uint64_t> dspare;
    bool spare_zeroed = false;
    bool trans = false;         // some rule reads it backward
    bool prev = false, prev_t = false;  // R minus D read forward / backward
    uint64_t rcount = 0, dcount = 0;
};
struct CsrRel {  // an EDB predicate in one direction
    Buf<uint64_t> row_ptr, mask, pairs_t;
    Buf<uint32_t> adj;
    bool built = false;
};

struct ChainRun {
    Ctx *ctx;
    const std::vector<ChainRule> &rules;
    uint32_t n_preds, domain, words;
    uint64_t cells;
    const std::vector<char> &idb;
    const std::vector<const uint64_t *> &keys;
    const std::vector<uint64_t> &rows;
    std::vector<BitRel> bit;       // by predicate (IDB only)
    std::vector<CsrRel> csr[2];    // by predicate: forward, backward (EDB only)
    Buf<uint64_t> T[2], TM[2];
    // partial delta counts: CHUNK iterations x predicates x SPREAD, and their sums
    static constexpr int CHUNK = 8;
    Buf<unsigned long long> counts, totals;
    int slot = 0;             // iteration slot of the chunk being queued
    bool speculative = false; // delta sizes of the queued iterations are not known yet
    // every iteration after the seed is fused for every head: the fused
    // products write whole rows, and retired delta rows need no clearing
    bool no_clear = false;
    unsigned long long *cnt_of(int p) { return counts.p + ((uint64_t)slot * n_preds + p) * SPREAD; }
    std::vector<int> idb_list;

    void fill0(Buf<uint64_t> &b, uint64_t n) { fill_u64(ctx, b.p, 0ull, n); }
    FillBatch zero{ctx};  // zero-fills gathered into one launch (flushed by setup and begin_iteration)
    void zero0(Buf<uint64_t> &b, uint64_t n) { zero.add(b.p, n); }

    // seed_rows: the seed writes R and D of the one IDB predicate whole
    // (k_seed_rows), so they are not zero-filled; nor is the candidate matrix
    // when every product is fused (each writes the rows it marks whole)
    void setup(bool seed_rows = false) {
        bit.resize(n_preds);
        csr[0].resize(n_preds);
        csr[1].resize(n_preds);
        size_t max_len = 0;
        for (const ChainRule &r : rules) {
            max_len = std::max(max_len, r.path.size());
            for (size_t j = 0; j < r.path.size(); ++j) {
                const ChainAtom &a = r.path[j];
                if (idb[a.pred]) {
                    if (a.backward) bit[a.pred].trans = true;
                    // an IDB atom with a later IDB atom reads R minus D when the delta sits there
                    for (size_t k = j + 1; k < r.path.size(); ++k)
                        if (idb[r.path[k].pred]) (a.backward ? bit[a.pred].prev_t : bit[a.pred].prev) = true;
                } else if (rows[a.pred]) {
                    csr[a.backward ? 1 : 0][a.pred].built = true;  // built below
                }
            }
        }
        for (uint32_t p = 0; p < n_preds; ++p) {
            if (!idb[p]) continue;
            idb_list.push_back((int)p);
            BitRel &b = bit[p];
            b.R = Buf<uint64_t>(ctx, cells);
            b.D = Buf<uint64_t>(ctx, cells);
            b.C = Buf<uint64_t>(ctx, cells);
            if (!seed_rows) {
                zero0(b.R, cells);
                zero0(b.D, cells);
            }
            b.rmask = Buf<uint64_t>(ctx, words); zero0(b.rmask, words);
            b.dmask[0] = Buf<uint64_t>(ctx, words); zero0(b.dmask[0], words);
            b.dmask[1] = Buf<uint64_t>(ctx, words); zero0(b.dmask[1], words);
            b.cmask = Buf<uint64_t>(ctx, words); zero0(b.cmask, words);
            if (b.trans) {
                b.RT = Buf<uint64_t>(ctx, cells); zero0(b.RT, cells);
                b.DT = Buf<uint64_t>(ctx, cells); zero0(b.DT, cells);
                b.rtmask = Buf<uint64_t>(ctx, words); zero0(b.rtmask, words);
                b.dtmask = Buf<uint64_t>(ctx, words); zero0(b.dtmask, words);
            }
            if (b.prev) {
                b.P = Buf<uint64_t>(ctx, cells); zero0(b.P, cells);
                b.pmask = Buf<uint64_t>(ctx, words); zero0(b.pmask, words);
            }
            if (b.prev_t) {
                b.PT = Buf<uint64_t>(ctx, cells); zero0(b.PT, cells);
                b.ptmask = Buf<uint64_t>(ctx, words); zero0(b.ptmask, words);
            }
            if (rows[p]) {  // initial contents of the head relation (also R minus D: D starts empty)
                zero.flush();  // the matrices are zero before the rows are OR-ed in
                const unsigned g = grid_for(rows[p], 256, 4096);
                hipLaunchKernelGGL(k_pairs_bits_mask, dim3(g), dim3(256), 0, ctx->stream, keys[p], rows[p], 1, words,
                                   b.R.p, b.rmask.p);
                if (b.trans)
                    hipLaunchKernelGGL(k_pairs_bits_mask, dim3(g), dim3(256), 0, ctx->stream, keys[p], rows[p], 0,
                                       words, b.RT.p, b.rtmask.p);
                if (b.prev)
                    hipLaunchKernelGGL(k_pairs_bits_mask, dim3(g), dim3(256), 0, ctx->stream, keys[p], rows[p], 1,
                                       words, b.P.p, b.pmask.p);
                if (b.prev_t)
                    hipLaunchKernelGGL(k_pairs_bits_mask, dim3(g), dim3(256), 0, ctx->stream, keys[p], rows[p], 0,
                                       words, b.PT.p, b.ptmask.p);
                XH_CHECK_HIP(hipGetLastError());
                b.rcount = rows[p];
            }
        }
        for (int dir = 0; dir < 2; ++dir)
            for (uint32_t p = 0; p < n_preds; ++p) {
                CsrRel &c = csr[dir][p];
                if (!c.built) continue;
                const uint64_t *pairs = keys[p];
                const uint64_t m = rows[p];
                if (dir == 1) {  // transposed: swap the columns and re-sort (rows stay unique)
                    c.pairs_t = Buf<uint64_t>(ctx, m);
                    Buf<uint64_t> alt(ctx, m);
                    swap_words(ctx, keys[p], m, c.pairs_t.p);
                    uint64_t *a = c.pairs_t.p, *b = alt.p;
                    radix_sort_u64(ctx, &a, &b, nullptr, nullptr, m);
                    if (a != c.pairs_t.p) std::swap(c.pairs_t.p, alt.p);
                    pairs = c.pairs_t.p;
                }
                c.row_ptr = Buf<uint64_t>(ctx, (uint64_t)domain + 1);
                c.adj = Buf<uint32_t>(ctx, m);
                c.mask = Buf<uint64_t>(ctx, words);
                pairs_csr(ctx, pairs, m, domain, c.row_ptr.p, c.adj.p);
                hipLaunchKernelGGL(k_csr_mask, dim3(grid_for(words, 256, 1024)), dim3(256), 0, ctx->stream,
                                   c.row_ptr.p, domain, words, c.mask.p);
                XH_CHECK_HIP(hipGetLastError());
            }
        if (max_len >= 3) {
            T[0] = Buf<uint64_t>(ctx, cells);
            TM[0] = Buf<uint64_t>(ctx, words);
        }
        if (max_len >= 4) {
            T[1] = Buf<uint64_t>(ctx, cells);
            TM[1] = Buf<uint64_t>(ctx, words);
        }
        counts = Buf<unsigned long long>(ctx, (uint64_t)CHUNK * n_preds * SPREAD);
        totals = Buf<unsigned long long>(ctx, (uint64_t)CHUNK * n_preds);
        if (!(seed_rows && all_fused()))
            for (int p : idb_list) zero0(bit[p].C, cells);
        zero.flush();
    }

    enum Use { FULL, DELTA, PREV };  // R, D, or R minus D
    // operand for atom a; false when it is known to be empty
    bool operand(const ChainAtom &a, Use use, Operand &op) {
        op = Operand{nullptr, nullptr, nullptr, nullptr};
        if (idb[a.pred]) {
            BitRel &b = bit[a.pred];
            const uint64_t n = use == FULL ? b.rcount : (use == DELTA ? b.dcount : b.rcount - b.dcount);
            if (n == 0 && !speculative) return false;  // (queued iterations: the masks skip empty rows)
            if (!a.backward) {
                op.bits = use == FULL ? b.R.p : (use == DELTA ? b.D.p : b.P.p);
                op.mask = use == FULL ? b.rmask.p : (use == DELTA ? b.dmask[b.dcur].p : b.pmask.p);
            } else {
                op.bits = use == FULL ? b.RT.p : (use == DELTA ? b.DT.p : b.PT.p);
                op.mask = use == FULL ? b.rtmask.p : (use == DELTA ? b.dtmask.p : b.ptmask.p);
            }
            return true;
        }
        if (rows[a.pred] == 0) return false;
        CsrRel &c = csr[a.backward ? 1 : 0][a.pred];
        op.row_ptr = c.row_ptr.p;
        op.adj = c.adj.p;
        op.mask = c.mask.p;
        return true;
    }

    template <bool LCSR, bool RCSR, bool ACC>
    void launch(const Operand &l, const Operand &r, uint64_t *o, uint64_t *om, unsigned long long *work) {
        hipLaunchKernelGGL((k_chain_product<LCSR, RCSR, ACC>), dim3(domain), dim3(PTB), words * sizeof(uint64_t),
                           ctx->stream, words, l, r, o, om, work);
    }
    // mode: OUT_ASSIGN (temporary), OUT_OR (candidates) or OUT_FUSED (new delta + R, CSR left only)
    void product(const Operand &l, const Operand &r, int mode, uint64_t *o, uint64_t *om, const FusedArgs &fz) {
        // algorithmic bytes: the rows each active block reads and writes, counted on the device
        Prof prof(ctx, XLOG_HIP_KERNEL_CHAIN_PRODUCT, 0.0);
        unsigned long long *w = prof.work(1.0);
        const bool lc = l.bits == nullptr, rc = r.bits == nullptr, acc = mode != OUT_ASSIGN;
        XH_REQUIRE(mode != OUT_FUSED || (lc && !rc), XLOG_HIP_INVALID_ARG, "chain bitmap: fused product needs a CSR left");
        if (mode == OUT_FUSED) {  // a wave per batch of rows
            const uint32_t batch = row_batch(domain);
            const uint32_t blocks = (domain + GW * batch - 1) / (GW * batch);
            hipLaunchKernelGGL(k_csr_gather_fused, dim3(blocks), dim3(GW * WAVE), 0, ctx->stream,
                               domain, words, batch, l, r, o, om, fz, w);
            XH_CHECK_HIP(hipGetLastError());
            return;
        }
        if (acc) {
            if (lc && rc) launch<true, true, true>(l, r, o, om, w);
            else if (lc) launch<true, false, true>(l, r, o, om, w);
            else if (rc) launch<false, true, true>(l, r, o, om, w);
            else launch<false, false, true>(l, r, o, om, w);
        } else {
            if (lc && rc) launch<true, true, false>(l, r, o, om, w);
            else if (lc) launch<true, false, false>(l, r, o, om, w);
            else if (rc) launch<false, true, false>(l, r, o, om, w);
            else launch<false, false, false>(l, r, o, om, w);
        }
        XH_CHECK_HIP(hipGetLastError());
    }

    // Candidates of rule r with the delta at atom `delta_at` (-1: none, every
    // atom full).  IDB atoms before the delta read R minus D and those after
    // it R: over all delta positions this covers each derivation with at
    // least one delta atom exactly once (at its first one), the same union as
    // delta-at-one-position, full-elsewhere, with smaller left operands.
    void eval_chain(const ChainRule &r, int delta_at, bool fused = false) {
        const size_t k = r.path.size();
        Operand ops[8];
        for (size_t j = 0; j < k; ++j) {
            const Use use = (int)j == delta_at ? DELTA : ((int)j < delta_at ? PREV : FULL);
            if (!operand(r.path[j], use, ops[j])) return;
        }
        BitRel &H = bit[r.head];
        if (k == 1) {
            const ChainAtom &a = r.path[0];
            if (idb[a.pred]) {
                hipLaunchKernelGGL(k_or_rows, dim3(domain), dim3(FTB), 0, ctx->stream, words, ops[0].bits,
                                   ops[0].mask, H.C.p, H.cmask.p);
            } else {
                hipLaunchKernelGGL(k_pairs_bits_mask, dim3(grid_for(rows[a.pred], 256, 4096)), dim3(256), 0,
                                   ctx->stream, keys[a.pred], rows[a.pred], a.backward ? 0 : 1, words, H.C.p,
                                   H.cmask.p);
            }
            XH_CHECK_HIP(hipGetLastError());
            return;
        }
        // the last product ORs into the candidates, or, fused, writes the new delta into them
        const int last_mode = fused ? OUT_FUSED : OUT_OR;
        const FusedArgs fz{H.R.p, H.rmask.p, cnt_of(r.head), no_clear ? 1u : 0u, no_clear ? H.dspare.p : nullptr,
                           words};
        uint64_t *last_mask = fused ? H.dmask[H.dcur ^ 1].p : H.cmask.p;
        if (!right_to_left(r)) {  // ((a1 a2) a3) ...
            Operand left = ops[0];
            for (size_t j = 1; j < k; ++j) {
                const bool last = j + 1 == k;
                uint64_t *o = last ? H.C.p : T[(j - 1) & 1].p;
                uint64_t *om = last ? last_mask : TM[(j - 1) & 1].p;
                if (!last) fill_u64(ctx, om, 0ull, words);
                product(left, ops[j], last ? last_mode : OUT_ASSIGN, o, om, fz);
                left = Operand{o, nullptr, nullptr, om};
            }
        } else {  // a1 (a2 (a3 ...))
            Operand right = ops[k - 1];
            for (size_t j = k - 1; j-- > 0;) {
                const bool last = j == 0;
                const size_t t = (k - 2 - j) & 1;
                uint64_t *o = last ? H.C.p : T[t].p;
                uint64_t *om = last ? last_mask : TM[t].p;
                if (!last) fill_u64(ctx, om, 0ull, words);
                product(ops[j], right, last ? last_mode : OUT_ASSIGN, o, om, fz);
                right = Operand{o, nullptr, nullptr, om};
            }
        }
        if (fused && no_clear) H.spare_zeroed = true;
    }

    // The variant can write its head's new delta directly (OUT_FUSED) when it
    // is the head's only variant this iteration, its last product has a CSR
    // left operand, and nothing else of the head is read or kept: no other
    // atom of the head in the body (the product updates R in place), no
    // transposes and no R-minus-delta copy to maintain.
    // Every IDB head has exactly one IDB occurrence over its rules, and that
    // variant can take the fused product.
    bool all_fused() const {
        std::vector<int> occ(n_preds, 0);
        for (const ChainRule &r : rules)
            for (size_t j = 0; j < r.path.size(); ++j)
                if (idb[r.path[j].pred]) ++occ[r.head];
        for (const ChainRule &r : rules)
            for (size_t j = 0; j < r.path.size(); ++j)
                if (idb[r.path[j].pred] && (occ[r.head] != 1 || !can_fuse(r, (int)j))) return false;
        for (int p : idb_list)
            if (occ[p] != 1) return false;
        return true;
    }

    bool can_fuse(const ChainRule &r, int delta_at) const {
        const BitRel &H = bit[r.head];
        if (H.trans || H.prev || r.path.size() < 2) return false;
        for (size_t j = 0; j < r.path.size(); ++j)
            if ((int)j != delta_at && r.path[j].pred == r.head) return false;
        const bool rtl = right_to_left(r);
        // left operand of the last product: atom 0 (right to left, or a two-atom chain)
        if (!(rtl || r.path.size() == 2) || idb[r.path[0].pred]) return false;
        // its right operand must be a bitmap: an intermediate, or atom 1 of a two-atom chain
        return rtl || idb[r.path[1].pred];
    }

    // A product whose right operand is a CSR relation expands adjacency lists
    // id by id (latency-bound); with a bitmap right operand every id is one
    // coalesced row gather.  Left to right puts every EDB atom after the first
    // on the right, right to left only the last one, so a chain with an EDB
    // atom strictly inside runs right to left.
    bool right_to_left(const ChainRule &r) const {
        for (size_t j = 1; j + 1 < r.path.size(); ++j)
            if (!idb[r.path[j].pred]) return true;
        return false;
    }

    // Before an iteration's products: clear the counts (of every queued
    // iteration, at the first) and, for every head whose delta a fused product
    // writes, the new delta's row mask (already clear when every iteration is
    // fused: the previous product cleared it).
    // The new delta's and the candidates' row masks of a non-fused head are
    // cleared here too (nothing reads them before its finalize), all in one launch.
    void begin_iteration(const std::vector<char> &fused) {
        if (slot == 0) zero.add(reinterpret_cast<uint64_t *>(counts.p), (uint64_t)CHUNK * n_preds * SPREAD);
        for (int p : idb_list) {
            bit[p].spare_zeroed = false;
            if (fused[p] && !no_clear) zero.add(bit[p].dmask[bit[p].dcur ^ 1].p, words);
            if (!fused[p]) {
                zero.add(bit[p].dmask[bit[p].dcur ^ 1].p, words);
                zero.add(bit[p].cmask.p, words);
            }
        }
        zero.flush();
    }

    // New deltas of every IDB predicate from its candidates (or, for fused
    // heads, already in the candidate matrix); returns their total.
    void finalize_all(const std::vector<char> &fused) {
        for (int p : idb_list) {
            BitRel &b = bit[p];
            uint64_t *dnew = b.dmask[b.dcur ^ 1].p;
            if (fused[p]) {
                // the new delta is in C: retire the old delta rows, then swap the two matrices
                if (!no_clear) {
                    hipLaunchKernelGGL(k_clear_rows, dim3(domain), dim3(FTB), 0, ctx->stream, words, b.D.p,
                                       b.dmask[b.dcur].p);
                    XH_CHECK_HIP(hipGetLastError());
                }
                std::swap(b.D.p, b.C.p);
                b.dcur ^= 1;
                if (no_clear) {  // the delta mask read this iteration becomes the spare, the cleared spare the next new one
                    if (!b.spare_zeroed) fill0(b.dspare, words);
                    std::swap(b.dmask[b.dcur ^ 1].p, b.dspare.p);
                }
                continue;
            }
            FinalizeArgs fa{b.C.p, b.cmask.p, b.R.p, b.rmask.p, b.D.p, b.dmask[b.dcur].p, dnew, b.P.p,
                            b.pmask.p, cnt_of(p), nullptr};
            {
                Prof prof(ctx, XLOG_HIP_KERNEL_CHAIN_FINALIZE, 0.0);
                fa.work = prof.work(1.0);  // bytes of the row words moved, counted on the device
                const uint32_t batch = row_batch(domain), blocks = (domain + GW * batch - 1) / (GW * batch);
                if (b.prev)
                    hipLaunchKernelGGL((k_chain_finalize<true>), dim3(blocks), dim3(GW * WAVE), 0, ctx->stream, domain,
                                       words, batch, fa);
                else
                    hipLaunchKernelGGL((k_chain_finalize<false>), dim3(blocks), dim3(GW * WAVE), 0, ctx->stream, domain,
                                       words, batch, fa);
                XH_CHECK_HIP(hipGetLastError());
            }
            if (b.trans) {
                fill_u64(ctx, b.dtmask.p, 0ull, words);
                Prof prof(ctx, XLOG_HIP_KERNEL_CHAIN_FINALIZE, 0.0);
                const dim3 g((words + TT_COLS - 1) / TT_COLS, (words + TT_WAVES - 1) / TT_WAVES);
                hipLaunchKernelGGL(k_transpose_delta, g, dim3(TT_WAVES * WAVE), 0, ctx->stream, domain, words, b.D.p,
                                   b.dmask[b.dcur].p, dnew, b.DT.p, b.dtmask.p, b.RT.p, b.rtmask.p, b.PT.p,
                                   b.ptmask.p, prof.work(1.0));
                XH_CHECK_HIP(hipGetLastError());
            }
            b.dcur ^= 1;
        }
    }

    // Sums and reads back the delta sizes of the `queued` iterations (one
    // copy, pinned staging when it fits) into sizes[i * n_preds + p].
    void read_counts(int queued, std::vector<uint64_t> &sizes) {
        const uint32_t n = (uint32_t)queued * n_preds;
        hipLaunchKernelGGL(k_sum_counts, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, counts.p, n, totals.p);
        XH_CHECK_HIP(hipGetLastError());
        sizes.resize(n);
        if (n <= 64) {
            ctx->read_scalars(totals.p, n);
            for (uint32_t i = 0; i < n; ++i) sizes[i] = ctx->host_scalars[i];
        } else {
            XH_CHECK_HIP(hipMemcpyAsync(sizes.data(), totals.p, n * sizeof(uint64_t), hipMemcpyDeviceToHost,
                                        ctx->stream));
            ctx->sync();
        }
    }

    // Applies iteration i's delta sizes; returns their total.
    uint64_t take_counts(const std::vector<uint64_t> &sizes, int i) {
        uint64_t total = 0;
        for (int p : idb_list) {
            const uint64_t n = sizes[(uint64_t)i * n_preds + p];
            bit[p].dcount = n;
            bit[p].rcount += n;
            total += n;
        }
        return total;
    }
};

}  // namespace

uint64_t chain_fixpoint_bytes(const std::vector<ChainRule> &rules, const std::vector<char> &idb, uint32_t domain) {
    const uint64_t words = ((uint64_t)domain + 63) / 64, cells = (uint64_t)domain * words;
    std::vector<char> trans(idb.size(), 0), prev(idb.size(), 0), prev_t(idb.size(), 0);
    size_t max_len = 0;
    for (const ChainRule &r : rules) {
        max_len = std::max(max_len, r.path.size());
        for (size_t j = 0; j < r.path.size(); ++j) {
            const ChainAtom &a = r.path[j];
            if (!idb[a.pred]) continue;
            if (a.backward) trans[a.pred] = 1;
            for (size_t k = j + 1; k < r.path.size(); ++k)
                if (idb[r.path[k].pred]) (a.backward ? prev_t : prev)[a.pred] = 1;
        }
    }
    uint64_t mats = (max_len >= 3) + (max_len >= 4);
    for (size_t p = 0; p < idb.size(); ++p)
        if (idb[p]) mats += (trans[p] ? 5 : 3) + prev[p] + prev_t[p];
    return mats * cells * 8;
}

void chain_fixpoint(Ctx *ctx, const std::vector<ChainRule> &rules, uint32_t n_preds, const std::vector<char> &idb,
                    const std::vector<const uint64_t *> &keys, const std::vector<uint64_t> &rows, uint32_t domain,
                    uint64_t max_iter, std::vector<uint64_t *> &out, std::vector<uint64_t> &out_n,
                    uint64_t *iterations, std::vector<uint64_t> &deltas) {
    XH_REQUIRE(domain >= 1 && domain <= MAX_DOMAIN, XLOG_HIP_UNSUPPORTED, "chain bitmap: domain must be 1..2^17");
    for (const ChainRule &r : rules)
        XH_REQUIRE(!r.path.empty() && r.path.size() <= 8 && idb[r.head], XLOG_HIP_INVALID_ARG,
                   "chain bitmap: bad rule");
    deltas.clear();
    out.assign(n_preds, nullptr);
    out_n.assign(n_preds, 0);
    const uint32_t words = (domain + 63) / 64;
    ChainRun run{ctx, rules, n_preds, domain, words, (uint64_t)domain * words, idb, keys, rows};
    // One IDB predicate H that starts empty and whose one exit rule (no IDB
    // atom) is a single EDB atom E read forward (transitive closure): the seed
    // is R = D = E, written whole by k_seed_rows with |E| known on the host.
    int seed_h = -1, seed_e = -1, n_idb = 0, n_exit = 0;
    for (uint32_t p = 0; p < n_preds; ++p)
        if (idb[p]) {
            ++n_idb;
            seed_h = (int)p;
        }
    for (const ChainRule &r : rules) {
        bool exit_rule = true;
        for (const ChainAtom &a : r.path) exit_rule = exit_rule && !idb[a.pred];
        if (!exit_rule) continue;
        ++n_exit;
        if (r.path.size() == 1 && !r.path[0].backward) seed_e = r.path[0].pred;
    }
    const bool seed_cand = n_idb == 1 && rows[seed_h] == 0 && n_exit == 1 && seed_e >= 0 && rows[seed_e] > 0;
    run.setup(seed_cand);
    // (a head read backward or as R minus D also needs its transposes and P seeded: the general seed)
    const bool seed_rows =
        seed_cand && !run.bit[seed_h].trans && !run.bit[seed_h].prev && !run.bit[seed_h].prev_t;
    if (seed_cand && !seed_rows) {
        run.fill0(run.bit[seed_h].R, run.cells);
        run.fill0(run.bit[seed_h].D, run.cells);
    }
    const std::vector<char> none(n_preds, 0);
    std::vector<uint64_t> sizes;
    if (seed_rows) {
        BitRel &b = run.bit[seed_h];
        const CsrRel &c = run.csr[0][seed_e];
        XH_REQUIRE(c.built, XLOG_HIP_INVALID_ARG, "chain bitmap: the exit relation has no CSR");
        hipLaunchKernelGGL(k_seed_rows, dim3(domain), dim3(FTB), words * sizeof(uint64_t), ctx->stream, words,
                           c.row_ptr.p, c.adj.p, b.R.p, b.D.p);
        XH_CHECK_HIP(hipGetLastError());
        XH_CHECK_HIP(hipMemcpyAsync(b.rmask.p, c.mask.p, words * sizeof(uint64_t), hipMemcpyDeviceToDevice,
                                    ctx->stream));
        XH_CHECK_HIP(hipMemcpyAsync(b.dmask[b.dcur ^ 1].p, c.mask.p, words * sizeof(uint64_t),
                                    hipMemcpyDeviceToDevice, ctx->stream));
        b.dcur ^= 1;
        sizes.assign(n_preds, 0);
        sizes[seed_h] = rows[seed_e];
    } else {
        // seed: every rule once against the initial relations
        run.begin_iteration(none);
        for (const ChainRule &r : rules) run.eval_chain(r, -1);
        run.finalize_all(none);
        run.read_counts(1, sizes);
    }
    deltas.push_back(run.take_counts(sizes, 0));
    // When every head takes one fused variant per iteration (transitive
    // closure), CHUNK iterations are queued per read-back: an iteration after
    // the fixpoint finds every delta row empty, derives nothing and counts 0,
    // so the queued iterations past it change no relation and are not reported.
    const bool chunked = run.all_fused();
    run.no_clear = chunked;
    if (chunked)
        for (int p : run.idb_list) {
            run.bit[p].dspare = Buf<uint64_t>(ctx, words);
            run.fill0(run.bit[p].dspare, words);
        }
    uint64_t it = 0;
    bool converged = false;
    std::vector<int> nvar(n_preds);
    std::vector<char> fused(n_preds);
    while (it < max_iter && !converged) {
        const int queue = chunked ? (int)std::min<uint64_t>(ChainRun::CHUNK, max_iter - it) : 1;
        for (int k = 0; k < queue; ++k) {
            run.slot = k;
            run.speculative = k > 0;
            if (k == 0) {
                // the variants of this iteration; a head with exactly one may take the fused product
                std::fill(nvar.begin(), nvar.end(), 0);
                std::fill(fused.begin(), fused.end(), 0);
                for (const ChainRule &r : rules)
                    for (size_t j = 0; j < r.path.size(); ++j)
                        if (idb[r.path[j].pred] && run.bit[r.path[j].pred].dcount) ++nvar[r.head];
                for (const ChainRule &r : rules)
                    for (size_t j = 0; j < r.path.size(); ++j)
                        if (idb[r.path[j].pred] && run.bit[r.path[j].pred].dcount && nvar[r.head] == 1)
                            fused[r.head] = run.can_fuse(r, (int)j);
                // every head's one variant is fusable: fused even when its input delta is empty now (its
                // queued iterations may find one non-empty, and C is not kept clear for other products)
                if (run.no_clear)
                    for (int p : run.idb_list) fused[p] = 1;
            }
            run.begin_iteration(fused);
            for (const ChainRule &r : rules)
                for (size_t j = 0; j < r.path.size(); ++j) {
                    const int p = r.path[j].pred;
                    if (!idb[p] || (!run.speculative && run.bit[p].dcount == 0)) continue;
                    run.eval_chain(r, (int)j, fused[r.head] != 0);
                }
            run.finalize_all(fused);
        }
        run.read_counts(queue, sizes);
        run.speculative = false;
        for (int k = 0; k < queue && !converged; ++k) {
            ++it;
            const uint64_t total = run.take_counts(sizes, k);
            deltas.push_back(total);
            converged = total == 0;
        }
    }
    *iterations = it;
    XH_REQUIRE(converged, XLOG_HIP_ITERATION_LIMIT,
               "Recursive SCC iteration limit (" + std::to_string(max_iter) + ") exceeded");
    // release the working matrices before the results are materialised
    for (int p : run.idb_list) {
        BitRel &b = run.bit[p];
        b.D = Buf<uint64_t>(); b.C = Buf<uint64_t>(); b.RT = Buf<uint64_t>(); b.DT = Buf<uint64_t>();
        b.P = Buf<uint64_t>(); b.PT = Buf<uint64_t>();
    }
    run.T[0] = Buf<uint64_t>();
    run.T[1] = Buf<uint64_t>();
    for (int p : run.idb_list)
        // R's bits are its initial rows plus every delta: rcount, with no read-back
        out_n[p] = bitmap_emit(ctx, run.bit[p].R.p, domain, words, &out[p], XLOG_HIP_KERNEL_CHAIN_EMIT,
                               run.bit[p].rcount);
}

}  // namespace xh
