// Dense factorized transitive-closure step for gfx950, and the bitmap helpers
// the dense fixpoint routes share.
//
// The reference's factorized delta (fj_delta_novel_u32_recorded,
// crates/xlog-cuda/src/provider/fj_delta.rs:117-490; kernels wcoj.cu:3811-3946)
// computes  novel[x] = (U_{y in delta[x]} edge[y]) \ R[x]  with a
// domain x domain bitmap, capped at a 2^14..2^16 domain
// (wcoj_dispatch.rs:176-186).  fj_delta_step keeps that one-step operator:
// R, delta and the result are V x V bit matrices and k_tc_step handles one
// source row x per block:
//   acc     = OR over set bits y of delta[x] of the adjacency list of y  (LDS)
//   new     = acc & ~R[x];  R[x] |= new;  next[x] = new
// The result is emitted row by row in (x, z) order, so it is sorted and unique
// by construction.  (Inside the fixpoint, transitive closure runs on the chain
// route of chain_bitmap.hip, which gathers delta rows instead.)
#include "internal.hpp"

namespace xh {

namespace {

constexpr int TB = 256;
constexpr int CHUNK_WORDS = 64;  // delta-row words compacted per round (<= 4096 set bits)
constexpr int UNROLL = 4;        // adjacency lists loaded together per thread

// row_ptr[v] = first index of sorted unique edges with source >= v
__global__ void k_row_ptr(const uint64_t *__restrict__ edges, uint64_t m, uint32_t nv, uint64_t *__restrict__ row_ptr) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t v = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; v <= nv; v += stride) {
        uint64_t key = v << 32, lo = 0, hi = m;
        while (lo < hi) {
            uint64_t mid = (lo + hi) >> 1;
            if (edges[mid] < key) lo = mid + 1; else hi = mid;
        }
        row_ptr[v] = lo;
    }
}

__global__ void k_adj(const uint64_t *__restrict__ edges, uint64_t m, uint32_t *__restrict__ adj) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < m; i += stride) adj[i] = (uint32_t)edges[i];
}

// Dynamic LDS: `words` u64 accumulator words for the row.
__global__ __launch_bounds__(TB) void k_tc_step(uint32_t nv, uint64_t words, const uint64_t *__restrict__ row_ptr,
                                                const uint32_t *__restrict__ adj, uint64_t *__restrict__ R,
                                                const uint64_t *__restrict__ D, uint64_t *__restrict__ N,
                                                const uint8_t *__restrict__ nz_cur, uint8_t *__restrict__ nz_next,
                                                unsigned long long *__restrict__ count) {
    extern __shared__ uint64_t s_acc[];
    __shared__ unsigned long long s_cnt;
    __shared__ uint64_t s_bits[CHUNK_WORDS];
    __shared__ uint32_t s_woff[CHUNK_WORDS + 1];
    __shared__ uint32_t s_y[CHUNK_WORDS * 64];
    const uint32_t x = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    if (!nz_cur[x]) {
        if (tid == 0) nz_next[x] = 0;
        return;
    }
    for (uint64_t w = tid; w < words; w += TB) s_acc[w] = 0ull;
    if (tid == 0) s_cnt = 0;
    const uint64_t *drow = D + (uint64_t)x * words;
    const uint64_t lt_mask = (1ull << lane) - 1ull;
    // The delta row is consumed CHUNK_WORDS words at a time: its set bits y are
    // compacted into s_y, then all threads expand adjacency lists of distinct
    // y's (balanced regardless of where the bits sit), UNROLL lists in flight.
    for (uint64_t c0 = 0; c0 < words; c0 += CHUNK_WORDS) {
        if (wave == 0) {
            uint64_t w = c0 + lane;
            uint64_t bits = w < words ? drow[w] : 0ull;
            uint32_t pc = (uint32_t)__popcll(bits), incl = pc;
#pragma unroll
            for (int o = 1; o < WAVE; o <<= 1) {
                uint32_t t = __shfl_up(incl, o, WAVE);
                if (lane >= o) incl += t;
            }
            s_bits[lane] = bits;
            s_woff[lane] = incl - pc;
            if (lane == WAVE - 1) s_woff[CHUNK_WORDS] = incl;
        }
        __syncthreads();
        const uint32_t T = s_woff[CHUNK_WORDS];
        if (T) {
            for (int j = wave; j < CHUNK_WORDS; j += TB / WAVE) {
                uint64_t bits = s_bits[j];
                if ((bits >> lane) & 1ull)
                    s_y[s_woff[j] + (uint32_t)__popcll(bits & lt_mask)] = (uint32_t)((c0 + j) * 64 + lane);
            }
            __syncthreads();
            for (uint32_t q = tid; q < T; q += UNROLL * TB) {
                uint64_t b[UNROLL], f[UNROLL];
#pragma unroll
                for (int u = 0; u < UNROLL; ++u) {
                    uint32_t qq = q + u * TB;
                    uint32_t y = qq < T ? s_y[qq] : 0u;
                    b[u] = qq < T ? row_ptr[y] : 0ull;
                    f[u] = qq < T ? row_ptr[y + 1] : 0ull;
                }
#pragma unroll
                for (int u = 0; u < UNROLL; ++u)
                    for (uint64_t e = b[u]; e < f[u]; ++e) {
                        uint32_t z = adj[e];
                        atomicOr((unsigned long long *)&s_acc[z >> 6], 1ull << (z & 63));
                    }
            }
        }
        __syncthreads();
    }
    uint64_t *rrow = R + (uint64_t)x * words;
    uint64_t *nrow = N + (uint64_t)x * words;
    unsigned long long local = 0;
    for (uint64_t w = tid; w < words; w += TB) {
        uint64_t r = rrow[w];
        uint64_t nw = s_acc[w] & ~r;
        nrow[w] = nw;
        if (nw) {
            rrow[w] = r | nw;
            local += (unsigned long long)__popcll(nw);
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) local += __shfl_xor(local, o, WAVE);
    if ((tid & 63) == 0 && local) atomicAdd(&s_cnt, local);
    __syncthreads();
    if (tid == 0) {
        nz_next[x] = s_cnt != 0;
        if (s_cnt) {
            atomicAdd(count, s_cnt);
            atomicAdd(count + 1, 1ull);  // rows with a non-empty next delta
        }
    }
}

__global__ void k_set_ull(unsigned long long *p, unsigned long long v) { *p = v; }

// Bit (x, z) of a domain x domain bitmap for every packed pair row; x is the
// high word when x_hi, else the low word.  Rows outside the domain are
// skipped (callers reject them before the launch).
__global__ void k_pairs_to_bits(const uint64_t *__restrict__ rows, uint64_t n, int x_hi, uint32_t domain,
                                uint64_t words, uint64_t *__restrict__ B, uint8_t *__restrict__ nz) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t e = rows[i];
        const uint32_t x = x_hi ? (uint32_t)(e >> 32) : (uint32_t)e;
        const uint32_t z = x_hi ? (uint32_t)e : (uint32_t)(e >> 32);
        if (x >= domain || z >= domain) continue;
        atomicOr((unsigned long long *)&B[(uint64_t)x * words + (z >> 6)], 1ull << (z & 63));
        if (nz) nz[x] = 1;
    }
}

// per-row popcount of R
__global__ __launch_bounds__(TB) void k_row_counts(const uint64_t *__restrict__ R, uint64_t words,
                                                   uint64_t *__restrict__ cnt) {
    __shared__ unsigned long long s;
    const uint32_t x = blockIdx.x;
    if (threadIdx.x == 0) s = 0;
    __syncthreads();
    unsigned long long local = 0;
    for (uint64_t w = threadIdx.x; w < words; w += TB) local += __popcll(R[(uint64_t)x * words + w]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) local += __shfl_xor(local, o, WAVE);
    if ((threadIdx.x & 63) == 0) atomicAdd(&s, local);
    __syncthreads();
    if (threadIdx.x == 0) cnt[x] = s;
}

// Both emits write row x's set bits as (x << 32 | z) starting at off[x] (a
// block per row); positions at or past cap (the allocation: the caller may
// size it from its own count) are not written.
//
// Rows of a few thousand tuples or fewer: each wave stores its words' tuples
// straight from the bits (lane b stores bit b, so a dense word is one
// contiguous 512-byte store), TB words per step of the block.
__global__ __launch_bounds__(TB) void k_emit_rows_direct(const uint64_t *__restrict__ R, uint64_t words,
                                                  const uint64_t *__restrict__ off, uint64_t *__restrict__ out,
                                                  uint64_t cap) {
    __shared__ uint64_t s_part[TB / WAVE];
    __shared__ uint64_t s_base;
    __shared__ uint64_t s_word[TB];
    __shared__ uint64_t s_woff[TB];
    const uint32_t x = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t *row = R + (uint64_t)x * words;
    if (tid == 0) s_base = off[x];
    __syncthreads();
    // chunks of TB words: each thread one word; block-exclusive scan of popcounts
    for (uint64_t c0 = 0; c0 < words; c0 += TB) {
        uint64_t w = c0 + tid;
        uint64_t bits = w < words ? row[w] : 0ull;
        uint64_t pc = (uint64_t)__popcll(bits), x_incl = pc;
#pragma unroll
        for (int o = 1; o < WAVE; o <<= 1) {
            uint64_t t = __shfl_up(x_incl, o, WAVE);
            if (lane >= o) x_incl += t;
        }
        if (lane == 63) s_part[wave] = x_incl;
        __syncthreads();
        uint64_t pre = 0, tot = 0;
        for (int q = 0; q < TB / WAVE; ++q) {
            if (q < wave) pre += s_part[q];
            tot += s_part[q];
        }
        s_word[tid] = bits;
        s_woff[tid] = s_base + pre + x_incl - pc;
        __syncthreads();
        // wave q writes words q*64 .. q*64+63 of the chunk, one word per step:
        // lane b stores bit b, so a dense word is one contiguous 512-byte store
        const uint64_t hi = (uint64_t)x << 32;
        const uint64_t lt_mask = (1ull << lane) - 1ull;
        for (int j = 0; j < WAVE; ++j) {
            const int t = wave * WAVE + j;
            const uint64_t wb = s_word[t];
            if (wb == 0ull) continue;
            const uint64_t pos = s_woff[t] + (uint64_t)__popcll(wb & lt_mask);
            if (((wb >> lane) & 1ull) && pos < cap) out[pos] = hi | (uint64_t)((c0 + t) * 64 + lane);
        }
        __syncthreads();
        if (tid == 0) s_base += tot;
        __syncthreads();
    }
}

// Dense rows (EMIT_STAGED_ROW tuples or more on average): the row is read in
// chunks of EMIT_TB words (a block scan of their popcounts gives each word's
// offset); a group of EMIT_G words is expanded into an LDS buffer (a wave per
// word, a lane per bit), and the block then writes the group's tuples with
// stores aligned to 128-byte lines (a word's tuples start at any 8-byte
// offset, so storing them straight from the expanding wave splits lines).
// Two buffers, one barrier per group: the expansion of group g + 2 follows
// the barrier of group g + 1, which every thread passes after writing group g
// out.
constexpr int EMIT_TB = 512, EMIT_G = 64;
constexpr uint64_t EMIT_STAGED_ROW = 8192;
__global__ __launch_bounds__(EMIT_TB) void k_emit_rows(const uint64_t *__restrict__ R, uint64_t words,
                                                       const uint64_t *__restrict__ off, uint64_t *__restrict__ out,
                                                       uint64_t cap) {
    constexpr int WAVES = EMIT_TB / WAVE, WPG = EMIT_G / WAVES;
    static_assert(EMIT_TB % EMIT_G == 0 && EMIT_G % WAVES == 0, "groups split evenly over the waves");
    __shared__ uint64_t s_word[EMIT_TB];
    __shared__ uint32_t s_woff[EMIT_TB + 1];  // offsets inside the chunk; [EMIT_TB]: the chunk's total
    __shared__ uint32_t s_part[WAVES];
    __shared__ uint64_t buf[2][EMIT_G * 64];
    const uint32_t x = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t *row = R + (uint64_t)x * words;
    const uint64_t hi = (uint64_t)x << 32;
    const uint64_t lt_mask = (1ull << lane) - 1ull;
    uint64_t cbase = off[x];  // output position of the chunk's first tuple
    int gi = 0;
    for (uint64_t c0 = 0; c0 < words; c0 += EMIT_TB) {
        const uint64_t w = c0 + tid;
        const uint64_t bits = w < words ? row[w] : 0ull;
        const uint32_t pc = (uint32_t)__popcll(bits);
        uint32_t incl = pc;
#pragma unroll
        for (int o = 1; o < WAVE; o <<= 1) {
            const uint32_t t = __shfl_up(incl, o, WAVE);
            if (lane >= o) incl += t;
        }
        if (lane == WAVE - 1) s_part[wave] = incl;
        __syncthreads();
        uint32_t pre = 0, tot = 0;
#pragma unroll
        for (int q = 0; q < WAVES; ++q) {
            if (q < wave) pre += s_part[q];
            tot += s_part[q];
        }
        s_word[tid] = bits;
        s_woff[tid] = pre + incl - pc;
        if (tid == 0) s_woff[EMIT_TB] = tot;
        __syncthreads();
        const uint64_t cw = words - c0 < (uint64_t)EMIT_TB ? words - c0 : (uint64_t)EMIT_TB;
        for (uint32_t g0 = 0; g0 < cw; g0 += EMIT_G, ++gi) {
            uint64_t *b = buf[gi & 1];
            const uint32_t gb = s_woff[g0], ge = s_woff[g0 + EMIT_G];
#pragma unroll
            for (int j = 0; j < WPG; ++j) {
                const uint32_t t = g0 + (uint32_t)(wave * WPG + j);
                const uint64_t wb = s_word[t];
                if ((wb >> lane) & 1ull)
                    b[s_woff[t] - gb + (uint32_t)__popcll(wb & lt_mask)] = hi | (uint64_t)((c0 + t) * 64 + lane);
            }
            __syncthreads();
            // the group's tuples go to [gs, gs + ge - gb); o starts at the 128-byte line holding gs
            const uint64_t gs = cbase + gb;
            const uint32_t lead = (uint32_t)(gs & 15u), end = lead + (ge - gb);
            uint64_t *o = out + (gs - lead);
            const uint64_t room = cap > gs - lead ? cap - (gs - lead) : 0;  // positions below cap
            const uint32_t lim = room < (uint64_t)end ? (uint32_t)room : end;
            for (uint32_t i = (uint32_t)tid; i < lim; i += EMIT_TB)
                if (i >= lead) o[i] = b[i - lead];
        }
        cbase += tot;
    }
}

}  // namespace

// One factorized delta step (the reference's fj_delta_novel_u32_recorded,
// crates/xlog-cuda/src/provider/fj_delta.rs:117-490): bitmaps of full R and
// of delta over the domain, one k_tc_step (novel = (U_{y in delta[x]}
// edge[y]) & ~R[x]), then the novel bitmap emitted row by row, which gives
// sorted unique (x, z) rows.
uint64_t fj_delta_step(Ctx *ctx, const uint64_t *delta, uint64_t nd, int delta_x_hi, const uint64_t *edge,
                       uint64_t ne, const uint64_t *full, uint64_t nf, int full_x_hi, uint32_t domain,
                       uint64_t **out) {
    *out = nullptr;
    if (nd == 0 || ne == 0 || domain == 0) return 0;
    const uint64_t words = ((uint64_t)domain + 63) / 64;
    XH_REQUIRE(words * 8 <= 64 * 1024, XLOG_HIP_UNSUPPORTED, "fj delta: domain too large for an LDS row");
    const uint64_t cells = (uint64_t)domain * words;
    Buf<uint64_t> R(ctx, cells), D(ctx, cells), N(ctx, cells);
    Buf<uint64_t> row_ptr(ctx, (uint64_t)domain + 1);
    Buf<uint32_t> adj(ctx, ne);
    const uint64_t nz_bytes = ((uint64_t)domain + 3) / 4 * 4;
    Buf<uint8_t> nz(ctx, nz_bytes), nz_next(ctx, nz_bytes);
    Buf<unsigned long long> cnt(ctx, 2);
    fill_u64(ctx, R.p, 0ull, cells);
    fill_u64(ctx, D.p, 0ull, cells);
    fill_u64(ctx, N.p, 0ull, cells);
    fill_u64(ctx, reinterpret_cast<uint64_t *>(cnt.p), 0ull, 2);
    fill_u32(ctx, reinterpret_cast<uint32_t *>(nz.p), 0u, nz_bytes / 4);
    if (nf)
        hipLaunchKernelGGL(k_pairs_to_bits, dim3(grid_for(nf, 256, 4096)), dim3(256), 0, ctx->stream, full, nf,
                           full_x_hi, domain, words, R.p, nullptr);
    hipLaunchKernelGGL(k_pairs_to_bits, dim3(grid_for(nd, 256, 4096)), dim3(256), 0, ctx->stream, delta, nd,
                       delta_x_hi, domain, words, D.p, nz.p);
    hipLaunchKernelGGL(k_row_ptr, dim3(grid_for((uint64_t)domain + 1, 256, 4096)), dim3(256), 0, ctx->stream, edge,
                       ne, domain, row_ptr.p);
    hipLaunchKernelGGL(k_adj, dim3(grid_for(ne, 256, 4096)), dim3(256), 0, ctx->stream, edge, ne, adj.p);
    XH_CHECK_HIP(hipGetLastError());
    {
        Prof prof(ctx, XLOG_HIP_KERNEL_TC_STEP, 32.0 * (double)cells);
        hipLaunchKernelGGL(k_tc_step, dim3(domain), dim3(TB), words * sizeof(uint64_t), ctx->stream, domain, words,
                           row_ptr.p, adj.p, R.p, D.p, N.p, nz.p, nz_next.p, cnt.p);
        XH_CHECK_HIP(hipGetLastError());
    }
    return bitmap_emit(ctx, N.p, domain, words, out, XLOG_HIP_KERNEL_TC_EMIT);
}

// CSR of sorted unique packed (src << 32) | dst rows with every id < nv:
// row_ptr[v] .. row_ptr[v + 1] index the destinations of v in adj.
void pairs_csr(Ctx *ctx, const uint64_t *pairs, uint64_t m, uint32_t nv, uint64_t *row_ptr, uint32_t *adj) {
    hipLaunchKernelGGL(k_row_ptr, dim3(grid_for((uint64_t)nv + 1, 256, 4096)), dim3(256), 0, ctx->stream, pairs, m, nv,
                       row_ptr);
    if (m) hipLaunchKernelGGL(k_adj, dim3(grid_for(m, 256, 4096)), dim3(256), 0, ctx->stream, pairs, m, adj);
    XH_CHECK_HIP(hipGetLastError());
}

// The set bits of an nv x words bitmap as sorted packed (x << 32) | z rows
// (row counts, a scan, then one block per row writing at its offset; rows
// of EMIT_STAGED_ROW tuples or more on average are staged in LDS).
uint64_t bitmap_emit(Ctx *ctx, const uint64_t *bits, uint32_t nv, uint64_t words, uint64_t **out, int prof_kind,
                     uint64_t known_total) {
    *out = nullptr;
    if (nv == 0 || known_total == 0) return 0;
    Buf<uint64_t> rc(ctx, (uint64_t)nv + 1);
    hipLaunchKernelGGL(k_row_counts, dim3(nv), dim3(TB), 0, ctx->stream, bits, words, rc.p);
    XH_CHECK_HIP(hipGetLastError());
    scan_u64_inplace(ctx, rc.p, nv, rc.p + nv);
    uint64_t total = known_total;
    if (total == UINT64_MAX) {
        ctx->read_scalars(rc.p + nv, 1);
        total = ctx->host_scalars[0];
    }
    if (total == 0) return 0;
    *out = static_cast<uint64_t *>(ctx->alloc(total * sizeof(uint64_t)));
    Prof prof(ctx, prof_kind, 8.0 * (double)total + 8.0 * (double)nv * (double)words);
    // XLOG_HIP_EMIT_STAGED_ROW (read at each emit) replaces the row size from which the staged emit runs
    uint64_t staged_row = EMIT_STAGED_ROW;
    if (const char *e = getenv("XLOG_HIP_EMIT_STAGED_ROW")) staged_row = strtoull(e, nullptr, 10);
    if (total >= staged_row * nv)
        hipLaunchKernelGGL(k_emit_rows, dim3(nv), dim3(EMIT_TB), 0, ctx->stream, bits, words, rc.p, *out, total);
    else
        hipLaunchKernelGGL(k_emit_rows_direct, dim3(nv), dim3(TB), 0, ctx->stream, bits, words, rc.p, *out, total);
    XH_CHECK_HIP(hipGetLastError());
    return total;
}

}  // namespace xh
