// C ABI of libxlog_hip: context, relation handles and operators.  Host code;
// the semi-naive fixpoint driver is in fixpoint.hip, the kernels in sort.hip,
// select.hip, join.hip, tc_bitmap.hip, chain_bitmap.hip and hash_set.hip.
#include "host.hpp"

#include <algorithm>
#include <array>
#include <chrono>
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <memory>

namespace xh {

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------
static thread_local std::string g_last_error;
void set_error(const std::string &msg) { g_last_error = msg; }

template <class F>
static xlog_hip_status guarded(F &&f) {
    try {
        f();
        g_last_error.clear();
        return XLOG_HIP_OK;
    } catch (const Error &e) {
        g_last_error = e.msg;
        return e.code;
    } catch (const std::bad_alloc &) {
        g_last_error = "host allocation failed";
        return XLOG_HIP_OOM;
    } catch (const std::exception &e) {
        g_last_error = e.what();
        return XLOG_HIP_DEVICE_ERROR;
    }
}

// ---------------------------------------------------------------------------
// pool
// ---------------------------------------------------------------------------
size_t Pool::round_up(size_t b) {
    if (b < 256) return 256;
    // four size classes per power of two
    int lg = 63 - __builtin_clzll(b);
    size_t q = (lg >= 2) ? (size_t)1 << (lg - 2) : 1;
    return (b + q - 1) / q * q;
}
void *Pool::alloc(size_t bytes) {
    size_t sz = round_up(bytes);
    // the budget bounds the live bytes, as the reference's GpuMemoryManager
    // (crates/xlog-cuda/src/memory.rs:756-770; MemoryBudget::with_limit aborts on exceed)
    if (budget_ && in_use_ + sz > budget_)
        throw Error{XLOG_HIP_OOM, "GPU memory budget exceeded: requested " + std::to_string(sz) + " bytes with " +
                                      std::to_string(in_use_) + " in use, budget " + std::to_string(budget_)};
    auto it = free_.find(sz);
    void *p = nullptr;
    if (it != free_.end()) {
        p = it->second;
        free_.erase(it);
        cached_ -= sz;
    } else {
        if (budget_ && in_use_ + cached_ + sz > budget_) trim();  // the footprint stays within the budget
        hipError_t e = hipMalloc(&p, sz);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            trim();
            e = hipMalloc(&p, sz);
            if (e != hipSuccess) {
                (void)hipGetLastError();
                throw Error{XLOG_HIP_OOM, "device allocation of " + std::to_string(sz) + " bytes failed"};
            }
        }
    }
    live_[p] = sz;
    in_use_ += sz;
    if (in_use_ > peak_) peak_ = in_use_;
    return p;
}
void Pool::free(void *p) {
    if (!p) return;
    auto it = live_.find(p);
    if (it == live_.end()) return;
    size_t sz = it->second;
    live_.erase(it);
    in_use_ -= sz;
    free_.emplace(sz, p);
    cached_ += sz;
}
void Pool::trim() {
    (void)hipDeviceSynchronize();
    for (auto &kv : free_) (void)hipFree(kv.second);
    free_.clear();
    cached_ = 0;
}
Pool::~Pool() {
    (void)hipDeviceSynchronize();
    for (auto &kv : free_) (void)hipFree(kv.second);
    for (auto &kv : live_) (void)hipFree(kv.first);
}

void Ctx::read_scalars(const void *dev, size_t count_u64) {
    XH_REQUIRE(count_u64 <= HOST_STAGE_U64, XLOG_HIP_INVALID_ARG, "read_scalars: more than the pinned staging holds");
    XH_CHECK_HIP(hipMemcpyAsync(host_scalars, dev, count_u64 * sizeof(uint64_t), hipMemcpyDeviceToHost, stream));
    sync();
}

// ---------------------------------------------------------------------------
// small kernels used only by the host layer
// ---------------------------------------------------------------------------
namespace {

__global__ void k_widen(const uint32_t *__restrict__ c0, uint64_t n, uint64_t *__restrict__ out) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = c0[i];
}

// device view of a relation's words (or of any packed word arrays)
struct RelView {
    const uint64_t *w[MAX_WORDS];
    int arity;
};
struct RelOut {
    uint64_t *w[MAX_WORDS];
};
// value of column c (0..arity-1) of row i
__device__ __forceinline__ uint32_t col_value(const RelView &v, int c, uint64_t i) {
    if (v.arity == 1) return (uint32_t)v.w[0][i];
    const uint64_t x = v.w[c >> 1][i];
    return (c & 1) ? (uint32_t)x : (uint32_t)(x >> 32);
}
// packs out_arity column values into the words of one output row
__device__ __forceinline__ void put_row(const RelOut &o, int out_arity, const uint32_t *v, uint64_t i) {
    if (out_arity == 1) {
        o.w[0][i] = v[0];
        return;
    }
    for (int k = 0; 2 * k < out_arity; ++k)
        o.w[k][i] = ((uint64_t)v[2 * k] << 32) | (2 * k + 1 < out_arity ? v[2 * k + 1] : 0u);
}

struct ProjSpec {
    int in_arity, out_arity;
    int cols[MAX_ARITY];
};
__global__ void k_project(RelView in, uint64_t n, ProjSpec s, RelOut out) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        uint32_t v[MAX_ARITY];
        for (int j = 0; j < s.out_arity; ++j) v[j] = col_value(in, s.cols[j], i);
        put_row(out, s.out_arity, v, i);
    }
}

__global__ void k_col_to_key(RelView in, int c, const uint32_t *__restrict__ perm, uint64_t n,
                             uint64_t *__restrict__ key) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        uint64_t r = perm ? perm[i] : i;
        key[i] = (uint64_t)col_value(in, c, r) << 32;
    }
}
__global__ void k_iota(uint32_t *p, uint64_t n) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = (uint32_t)i;
}
__global__ void k_iota64(uint64_t *p, uint64_t n) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = i;
}
__global__ void k_gather(const uint64_t *__restrict__ in, const uint32_t *__restrict__ perm, uint64_t n,
                         uint64_t *__restrict__ out) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = in[perm[i]];
}
// group-start flags over sorted rows for the given key columns
__global__ void k_group_flags(RelView in, ProjSpec keys, uint64_t n, uint8_t *__restrict__ flags) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        bool f = (i == 0);
        if (!f)
            for (int j = 0; j < keys.out_arity; ++j)
                if (col_value(in, keys.cols[j], i) != col_value(in, keys.cols[j], i - 1)) f = true;
        flags[i] = f;
    }
}
__global__ void k_col_unsorted(RelView in, int c, uint64_t n, uint32_t *flag) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i + 1 < n; i += stride)
        if (col_value(in, c, i) > col_value(in, c, i + 1)) *flag = 1u;
}
// The largest word of n packed rows into *mx (atomicMax: *mx starts at 0 or
// at an earlier maximum).  One atomic per block; launched with at most
// 1024 blocks of 256 threads (MAX_LAUNCH_1D), so the atomics on the one
// address stay few.
__global__ __launch_bounds__(256) void k_max_u32_of_packed(const uint64_t *__restrict__ k, uint64_t n,
                                                           unsigned int *mx) {
    __shared__ unsigned int s_m[4];
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    unsigned int m = 0;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        uint64_t x = k[i];
        unsigned a = (unsigned)(x >> 32), b = (unsigned)x;
        m = max(m, max(a, b));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = max(m, (unsigned)__shfl_xor((int)m, o, 64));
    if ((threadIdx.x & 63) == 0) s_m[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) atomicMax(mx, max(max(s_m[0], s_m[1]), max(s_m[2], s_m[3])));
}
__global__ void k_u64_to_u32(const uint64_t *__restrict__ in, uint64_t n, uint32_t *__restrict__ out) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = (uint32_t)in[i];
}

}  // namespace

// defined in join.hip / tc_bitmap.hip
uint64_t join_probe_general(Ctx *ctx, const uint64_t *probe, uint64_t n, int pcol, const RunIndex &ix,
                            const uint32_t *payload, int out_arity, const int oc[4], uint64_t **out0,
                            uint64_t **out1);
void join_match_flags(Ctx *ctx, const uint64_t *probe, uint64_t n, int pcol, const RunIndex &ix, int want,
                      uint8_t *flags);

#define LAUNCH_1D(kern, n, ...)                                                                             \
    do {                                                                                                    \
        if ((n) > 0) {                                                                                      \
            hipLaunchKernelGGL(kern, dim3(grid_for((n), 256, 16384)), dim3(256), 0, ctx->stream, __VA_ARGS__); \
            XH_CHECK_HIP(hipGetLastError());                                                                \
        }                                                                                                   \
    } while (0)
// LAUNCH_1D with at most 1024 blocks (grid-stride reductions into one word)
#define MAX_LAUNCH_1D(kern, n, ...)                                                                         \
    do {                                                                                                    \
        if ((n) > 0) {                                                                                      \
            hipLaunchKernelGGL(kern, dim3(grid_for((n), 256, 1024)), dim3(256), 0, ctx->stream, __VA_ARGS__);  \
            XH_CHECK_HIP(hipGetLastError());                                                                \
        }                                                                                                   \
    } while (0)

// ---------------------------------------------------------------------------
// relations
// ---------------------------------------------------------------------------
xlog_hip_rel *rel_new(Ctx *ctx, uint32_t arity, uint64_t cap) {
    XH_REQUIRE(arity >= 1 && arity <= MAX_ARITY, XLOG_HIP_INVALID_ARG, "relation arity must be 1..8");
    std::unique_ptr<xlog_hip_rel> r(new xlog_hip_rel());
    r->ctx = ctx;
    r->arity = arity;
    r->cap = cap;
    if (cap) {
        try {
            for (int k = 0; k < r->nwords(); ++k) r->w[k] = static_cast<uint64_t *>(ctx->alloc(cap * sizeof(uint64_t)));
        } catch (...) {
            for (int k = 0; k < MAX_WORDS; ++k) ctx->free(r->w[k]);
            throw;
        }
    }
    return r.release();
}
void rel_free(xlog_hip_rel *r) {
    if (!r) return;
    if (r->ctx)
        for (int k = 0; k < MAX_WORDS; ++k) r->ctx->free(r->w[k]);
    delete r;
}
static RelView view_of(const xlog_hip_rel *r) {
    RelView v{{r->w[0], r->w[1], r->w[2], r->w[3]}, (int)r->arity};
    return v;
}
static RelOut out_of(xlog_hip_rel *r) {
    RelOut o{{r->w[0], r->w[1], r->w[2], r->w[3]}};
    return o;
}
// (a, b) words -> (word h0, word h1) words of n packed pairs (h in {0, 1}: the
// high or the low word of the input)
void project_pairs(Ctx *ctx, const uint64_t *in, uint64_t n, int h0, int h1, uint64_t *out) {
    ProjSpec s{2, 2, {h0, h1, 0, 0, 0, 0, 0, 0}};
    RelView v{{in, nullptr, nullptr, nullptr}, 2};
    RelOut o{{out, nullptr, nullptr, nullptr}};
    LAUNCH_1D(k_project, n, v, n, s, o);
}
void max_u32_of_packed(Ctx *ctx, const uint64_t *k, uint64_t n, unsigned int *mx) {
    MAX_LAUNCH_1D(k_max_u32_of_packed, n, k, n, mx);
}
// adopt device buffers (ownership moves to the relation)
xlog_hip_rel *rel_adopt(Ctx *ctx, uint32_t arity, uint64_t rows, uint64_t *w0, uint64_t *w1, uint32_t flags) {
    xlog_hip_rel *r = new xlog_hip_rel();
    r->ctx = ctx;
    r->arity = arity;
    r->rows = rows;
    r->cap = rows;
    r->w[0] = w0;
    r->w[1] = w1;
    r->flags = flags;
    return r;
}
// packs device-resident u32 columns (arity 1..8) into the words of r
static void pack_device_columns(Ctx *ctx, const uint32_t *const *cols, uint32_t arity, uint64_t rows, xlog_hip_rel *r) {
    if (!rows) return;
    if (arity == 1) {
        LAUNCH_1D(k_widen, rows, cols[0], rows, r->w[0]);
        return;
    }
    for (int k = 0; k < words_for(arity); ++k)
        pack_columns(ctx, cols[2 * k], 2u * k + 1 < arity ? cols[2 * k + 1] : nullptr, rows, r->w[k]);
}
// adopt all words (ownership moves to the relation)
static xlog_hip_rel *rel_adopt_words(Ctx *ctx, uint32_t arity, uint64_t rows, uint64_t *const *w, uint32_t flags) {
    xlog_hip_rel *r = rel_adopt(ctx, arity, rows, w[0], w[1], flags);
    r->w[2] = w[2];
    r->w[3] = w[3];
    return r;
}
void copy_d2d(Ctx *ctx, uint64_t *dst, const uint64_t *src, uint64_t n) {
    if (n) XH_CHECK_HIP(hipMemcpyAsync(dst, src, n * sizeof(uint64_t), hipMemcpyDeviceToDevice, ctx->stream));
}
static xlog_hip_rel *rel_clone(Ctx *ctx, const xlog_hip_rel *in) {
    xlog_hip_rel *r = rel_new(ctx, in->arity, in->rows);
    r->rows = in->rows;
    r->flags = in->flags;
    for (int k = 0; k < in->nwords(); ++k) copy_d2d(ctx, r->w[k], in->w[k], in->rows);
    return r;
}

uint64_t read_count(Ctx *ctx, const uint64_t *d) {
    ctx->read_scalars(d, 1);
    return ctx->host_scalars[0];
}

uint64_t *alloc_keys(Ctx *ctx, uint64_t n) {
    return static_cast<uint64_t *>(ctx->alloc((n ? n : 1) * sizeof(uint64_t)));
}

std::vector<Bags> bags_per_pred(Ctx *ctx, uint32_t n) {
    std::vector<Bags> r;
    r.reserve(n);
    for (uint32_t i = 0; i < n; ++i) r.emplace_back(ctx);
    return r;
}

// ---------------------------------------------------------------------------
// sorting helpers
// ---------------------------------------------------------------------------

// Sort a u64 key array of any length; the result is returned in a buffer
// owned by the caller (either `keys` itself or a new one).  With keys_owned
// the call consumes `keys`: it is either returned or freed.
// digit_lo / digit_hi restrict the sort to 8-bit digits [lo, hi) (4..8 = by
// the high word only, stable otherwise).
uint64_t *sort_keys(Ctx *ctx, uint64_t *keys, uint64_t n, bool keys_owned, int digit_lo, int digit_hi,
                    uint32_t known_digits, bool *whole) {
    if (whole) *whole = false;
    // a consumed input is freed if an error unwinds from here
    Owned in_guard(ctx, keys_owned ? keys : nullptr);
    if (n < 2) {
        if (keys_owned || n == 0) return in_guard.release();
        uint64_t *c = static_cast<uint64_t *>(ctx->alloc(n * sizeof(uint64_t)));
        copy_d2d(ctx, c, keys, n);
        return c;
    }
    const uint64_t CHUNK = 1ull << 29;
    if (n < (1ull << 30)) {
        Owned ga(ctx, keys_owned ? in_guard.release() : alloc_keys(ctx, n));
        Owned gb(ctx, alloc_keys(ctx, n));
        uint64_t *a = ga.p, *b = gb.p;
        uint32_t *v0 = nullptr, *v1 = nullptr;
        // without keys_owned the first pass reads the caller's keys; both ping-pong buffers are ours
        radix_sort_u64(ctx, &a, &b, &v0, &v1, n, digit_lo, digit_hi, keys_owned ? nullptr : keys, known_digits,
                       nullptr, whole);
        ga.release();
        gb.release();
        ctx->free(b);
        return a;
    }
    XH_REQUIRE(digit_lo == 0 && digit_hi == 8, XLOG_HIP_UNSUPPORTED, "partial-key sort above 2^30 keys");
    // chunked: sort pieces of 2^29 then merge pairwise
    Owned ga(ctx, keys_owned ? in_guard.release() : alloc_keys(ctx, n));
    uint64_t *a = ga.p;
    if (!keys_owned) copy_d2d(ctx, a, keys, n);
    Owned gb(ctx, alloc_keys(ctx, n));
    uint64_t *b = gb.p;
    std::vector<std::pair<uint64_t, uint64_t>> runs;
    for (uint64_t s = 0; s < n; s += CHUNK) {
        uint64_t len = std::min(CHUNK, n - s);
        uint64_t *ka = a + s, *kb = b + s;
        uint32_t *v0 = nullptr, *v1 = nullptr;
        radix_sort_u64(ctx, &ka, &kb, &v0, &v1, len, 0, 8, nullptr, known_digits);
        if (ka != a + s) copy_d2d(ctx, a + s, ka, len);
        runs.push_back({s, len});
    }
    uint64_t *src = a, *dst = b;
    while (runs.size() > 1) {
        std::vector<std::pair<uint64_t, uint64_t>> next;
        for (size_t i = 0; i < runs.size(); i += 2) {
            if (i + 1 < runs.size()) {
                merge_sorted(ctx, src + runs[i].first, runs[i].second, src + runs[i + 1].first, runs[i + 1].second,
                             dst + runs[i].first);
                next.push_back({runs[i].first, runs[i].second + runs[i + 1].second});
            } else {
                copy_d2d(ctx, dst + runs[i].first, src + runs[i].first, runs[i].second);
                next.push_back(runs[i]);
            }
        }
        runs.swap(next);
        std::swap(src, dst);
    }
    ga.release();
    gb.release();
    ctx->free(dst);
    return src;
}

// sorted (any) keys -> unique keys in a new buffer; returns count
static uint64_t unique_keys(Ctx *ctx, const uint64_t *sorted, uint64_t n, uint64_t **out) {
    Owned o(ctx, alloc_keys(ctx, n));
    Buf<uint64_t> cnt(ctx, 1);
    select_unique(ctx, sorted, n, o.p, cnt.p);
    const uint64_t c = read_count(ctx, cnt.p);
    *out = o.release();
    return c;
}

// Sorted unique copy of n keys (the caller's buffer is left as it is): returns
// the count, *out is a new buffer.  A large input whose high word splits it
// into short runs gets its unique keys from the fused short-run pass.
// known_digits: the digits the keys may vary in (0: unknown, the histograms decide)
void sort_unique_keys_async(Ctx *ctx, const uint64_t *keys, uint64_t n, uint64_t **out, uint64_t *d_count,
                            uint32_t known_digits) {
    if (n >= 2 && n < (1ull << 30)) {
        Owned ga(ctx, alloc_keys(ctx, n)), gb(ctx, alloc_keys(ctx, n));
        uint64_t *a = ga.p, *b = gb.p;
        uint32_t *v0 = nullptr, *v1 = nullptr;
        SortUnique uq;
        radix_sort_u64(ctx, &a, &b, &v0, &v1, n, 0, 8, keys, known_digits, &uq);
        ga.release();
        gb.release();
        Owned sorted(ctx, a), other(ctx, b);
        if (uq.done) {
            fill_u64(ctx, d_count, uq.count, 1);
            *out = sorted.release();
            return;
        }
        select_unique(ctx, a, n, b, d_count);
        *out = other.release();
        return;
    }
    uint64_t *s = sort_keys(ctx, const_cast<uint64_t *>(keys), n, false, 0, 8, known_digits);
    Owned gs(ctx, s != keys ? s : nullptr);
    Owned o(ctx, alloc_keys(ctx, n));
    select_unique(ctx, s, n, o.p, d_count);
    *out = o.release();
}
// The same with the count read back (returned).
static uint64_t sort_unique_keys(Ctx *ctx, const uint64_t *keys, uint64_t n, uint64_t **out) {
    Buf<uint64_t> cnt(ctx, 1);
    sort_unique_keys_async(ctx, keys, n, out, cnt.p);
    return read_count(ctx, cnt.p);
}

// Canonical (sorted, unique) copy of the packed keys of an arity<=2 relation
// or the relation's own buffer when it is already canonical (borrowed = true).
static void canonical_keys(Ctx *ctx, const xlog_hip_rel *r, Canon &c) {
    c.ctx = ctx;
    if (r->flags & REL_CANONICAL) {
        c.k = r->w[0];
        c.n = r->rows;
        return;
    }
    uint64_t *u;
    c.n = sort_unique_keys(ctx, r->w[0], r->rows, &u);
    c.owned = u;
    c.k = u;
}

// Stable permutation sorting rows of any arity by key_cols (most significant
// first): LSD over the key columns, one stable 32-bit radix sort per column.
static uint32_t *sort_perm(Ctx *ctx, const xlog_hip_rel *in, const std::vector<int> &cols) {
    uint64_t n = in->rows;
    XH_REQUIRE(n < (1ull << 30), XLOG_HIP_CAPACITY_OVERFLOW, "sort: keyed sort limited to 2^30 rows");
    uint32_t *perm = static_cast<uint32_t *>(ctx->alloc(n * sizeof(uint32_t)));
    uint32_t *perm2 = static_cast<uint32_t *>(ctx->alloc(n * sizeof(uint32_t)));
    uint64_t *k0 = static_cast<uint64_t *>(ctx->alloc(n * sizeof(uint64_t)));
    uint64_t *k1 = static_cast<uint64_t *>(ctx->alloc(n * sizeof(uint64_t)));
    LAUNCH_1D(k_iota, n, perm, n);
    for (int i = (int)cols.size() - 1; i >= 0; --i) {
        LAUNCH_1D(k_col_to_key, n, view_of(in), cols[i], perm, n, k0);
        uint64_t *ka = k0, *kb = k1;
        uint32_t *va = perm, *vb = perm2;
        // the column sits in the high word (low word zero): digits 4..8 only
        radix_sort_u64(ctx, &ka, &kb, &va, &vb, n, 4, 8);
        k0 = ka; k1 = kb;
        perm = va; perm2 = vb;
    }
    ctx->free(perm2);
    ctx->free(k0);
    ctx->free(k1);
    return perm;
}

static xlog_hip_rel *gather_rel(Ctx *ctx, const xlog_hip_rel *in, const uint32_t *perm) {
    xlog_hip_rel *r = rel_new(ctx, in->arity, in->rows);
    r->rows = in->rows;
    uint64_t n = in->rows;
    for (int k = 0; k < in->nwords(); ++k) LAUNCH_1D(k_gather, n, in->w[k], perm, n, r->w[k]);
    return r;
}

static bool is_full_key(const xlog_hip_rel *in, const std::vector<int> &cols) {
    std::vector<int> uniq;
    for (int c : cols)
        if (std::find(uniq.begin(), uniq.end(), c) == uniq.end()) uniq.push_back(c);
    if (uniq.size() != in->arity) return false;
    for (size_t i = 0; i < uniq.size(); ++i)
        if (uniq[i] != (int)i) return false;
    return true;
}

static std::vector<int> check_cols(const xlog_hip_rel *in, const uint32_t *cols, uint32_t n) {
    XH_REQUIRE(n == 0 || cols, XLOG_HIP_INVALID_ARG, "key column list is NULL");
    std::vector<int> v;
    for (uint32_t i = 0; i < n; ++i) {
        XH_REQUIRE(cols[i] < in->arity, XLOG_HIP_INVALID_ARG,
                   "key column " + std::to_string(cols[i]) + " out of range for arity " + std::to_string(in->arity));
        v.push_back((int)cols[i]);
    }
    return v;
}

static xlog_hip_rel *op_sort(Ctx *ctx, const xlog_hip_rel *in, const std::vector<int> &cols) {
    if (in->rows < 2 || cols.empty()) return rel_clone(ctx, in);
    if (in->arity <= 2 && is_full_key(in, cols)) {
        if (in->flags & REL_CANONICAL) return rel_clone(ctx, in);
        uint64_t *s = sort_keys(ctx, in->w[0], in->rows, false);
        return rel_adopt(ctx, in->arity, in->rows, s, nullptr, 0);
    }
    uint32_t *perm = sort_perm(ctx, in, cols);
    xlog_hip_rel *r = gather_rel(ctx, in, perm);
    ctx->free(perm);
    return r;
}

static xlog_hip_rel *compact_rel(Ctx *ctx, const xlog_hip_rel *in, const uint8_t *flags) {
    Buf<uint64_t> cnt(ctx, in->nwords());
    Buf<uint64_t> o[MAX_WORDS];
    for (int k = 0; k < in->nwords(); ++k) {
        o[k] = Buf<uint64_t>(ctx, in->rows ? in->rows : 1);
        select_flags(ctx, in->w[k], flags, in->rows, o[k].p, cnt.p + k);
    }
    uint64_t n = read_count(ctx, cnt.p);
    uint64_t *w[MAX_WORDS] = {o[0].release(), o[1].release(), o[2].release(), o[3].release()};
    return rel_adopt_words(ctx, in->arity, n, w, 0);
}

static xlog_hip_rel *op_dedup_full(Ctx *ctx, const xlog_hip_rel *in) {
    if (in->flags & REL_CANONICAL) return rel_clone(ctx, in);
    if (in->arity <= 2) {
        uint64_t *u;
        const uint64_t n = sort_unique_keys(ctx, in->w[0], in->rows, &u);
        return rel_adopt(ctx, in->arity, n, u, nullptr, REL_CANONICAL);
    }
    std::vector<int> all;
    for (uint32_t c = 0; c < in->arity; ++c) all.push_back((int)c);
    xlog_hip_rel *s = op_sort(ctx, in, all);
    Buf<uint8_t> flags(ctx, s->rows ? s->rows : 1);
    ProjSpec ks{(int)s->arity, (int)s->arity, {0, 1, 2, 3, 4, 5, 6, 7}};
    LAUNCH_1D(k_group_flags, s->rows, view_of(s), ks, s->rows, flags.p);
    xlog_hip_rel *r = compact_rel(ctx, s, flags.p);
    rel_free(s);
    r->flags = REL_CANONICAL;
    return r;
}

static xlog_hip_rel *op_dedup(Ctx *ctx, const xlog_hip_rel *in, const std::vector<int> &cols) {
    if (is_full_key(in, cols)) return op_dedup_full(ctx, in);
    XH_REQUIRE(!cols.empty(), XLOG_HIP_INVALID_ARG, "dedup needs at least one key column");
    xlog_hip_rel *s = op_sort(ctx, in, cols);
    Buf<uint8_t> flags(ctx, s->rows ? s->rows : 1);
    std::vector<int> keys;  // distinct key columns (at most the arity)
    for (int c : cols)
        if (std::find(keys.begin(), keys.end(), c) == keys.end()) keys.push_back(c);
    ProjSpec ks{(int)s->arity, (int)keys.size(), {0, 0, 0, 0, 0, 0, 0, 0}};
    for (int j = 0; j < ks.out_arity; ++j) ks.cols[j] = keys[j];
    LAUNCH_1D(k_group_flags, s->rows, view_of(s), ks, s->rows, flags.p);
    xlog_hip_rel *r = compact_rel(ctx, s, flags.p);
    rel_free(s);
    return r;
}

static xlog_hip_rel *op_union_many(Ctx *ctx, const xlog_hip_rel *const *ins, uint32_t n) {
    XH_REQUIRE(n >= 1 && ins, XLOG_HIP_INVALID_ARG, "union needs at least one input");
    uint32_t arity = ins[0]->arity;
    uint64_t total = 0;
    for (uint32_t i = 0; i < n; ++i) {
        XH_REQUIRE(ins[i], XLOG_HIP_INVALID_ARG, "union input is NULL");
        XH_REQUIRE(ins[i]->arity == arity, XLOG_HIP_TYPE_MISMATCH, "union inputs have different arity");
        total += ins[i]->rows;
    }
    if (arity <= 2 && n == 2 && (ins[0]->flags & ins[1]->flags & REL_CANONICAL)) {
        uint64_t *m = static_cast<uint64_t *>(ctx->alloc((total ? total : 1) * sizeof(uint64_t)));
        merge_sorted(ctx, ins[0]->w[0], ins[0]->rows, ins[1]->w[0], ins[1]->rows, m);
        uint64_t *u;
        uint64_t cnt = unique_keys(ctx, m, total, &u);
        ctx->free(m);
        return rel_adopt(ctx, arity, cnt, u, nullptr, REL_CANONICAL);
    }
    xlog_hip_rel *cat = rel_new(ctx, arity, total);
    cat->rows = total;
    uint64_t off = 0;
    for (uint32_t i = 0; i < n; ++i) {
        for (int k = 0; k < cat->nwords(); ++k) copy_d2d(ctx, cat->w[k] + off, ins[i]->w[k], ins[i]->rows);
        off += ins[i]->rows;
    }
    xlog_hip_rel *r = op_dedup_full(ctx, cat);
    rel_free(cat);
    return r;
}

static xlog_hip_rel *op_diff(Ctx *ctx, const xlog_hip_rel *a, const xlog_hip_rel *b) {
    XH_REQUIRE(a->arity == b->arity, XLOG_HIP_TYPE_MISMATCH, "diff inputs have different arity");
    XH_REQUIRE(a->arity <= 2, XLOG_HIP_UNSUPPORTED, "diff: arity above 2 is not supported");
    Canon ca, cb;
    canonical_keys(ctx, a, ca);
    canonical_keys(ctx, b, cb);
    uint64_t *o = static_cast<uint64_t *>(ctx->alloc((ca.n ? ca.n : 1) * sizeof(uint64_t)));
    Buf<uint64_t> cnt(ctx, 1);
    select_unique_diff(ctx, ca.k, ca.n, cb.k, cb.n, o, cnt.p);
    uint64_t n = read_count(ctx, cnt.p);
    return rel_adopt(ctx, a->arity, n, o, nullptr, REL_CANONICAL);
}

// The build side of a join on a key list, folded into dense ids (see
// op_join_keys): one sorted unique u64 key array per folding step, in which
// the probe side's keys are ranked, and the run index over (id << 32) | row.
struct KeyFold {
    std::vector<Buf<uint64_t>> dict;
    std::vector<uint64_t> dict_n;
    JoinIndex J;
};
}  // namespace xh
// Reusable join index handle of the C ABI (one build, many probes): one key
// column of a relation of at most two columns is indexed directly (J, runs of
// that column's values, payload = the other column); any other key list is
// folded (F).
struct xlog_hip_join_index {
    xh::Ctx *ctx = nullptr;
    xh::JoinIndex J;
    std::unique_ptr<xh::KeyFold> F;
    uint32_t arity = 0;
    std::vector<uint32_t> keys;
    uint64_t rows = 0;
};
namespace xh {
// payload_sorted: the payload order inside a run is ascending; unique_rows
// (implies payload_sorted): duplicate (key, payload) rows are dropped, so a
// run's payloads are distinct (set-semantics callers only).
void build_join_index(Ctx *ctx, const uint64_t *keys, uint64_t n, uint32_t arity, int col, bool canonical,
                      JoinIndex &J, bool payload_sorted, bool unique_rows) {
    if (unique_rows) payload_sorted = true;
    J.n = n;
    uint64_t *sk = nullptr;
    bool own = false;
    // Runs of equal keys must be contiguous; unless payload_sorted is asked
    // for, the payload order inside a run is irrelevant and only the key word
    // (digits 4..7) is sorted.
    const int dlo = payload_sorted ? 0 : 4;
    if (arity == 1) {
        // (c0 << 32) | 0
        sk = static_cast<uint64_t *>(ctx->alloc((n ? n : 1) * sizeof(uint64_t)));
        swap_words(ctx, keys, n, sk);
        own = true;
        sk = sort_keys(ctx, sk, n, true, 4, 8);
    } else if (col == 0) {
        if (canonical) sk = const_cast<uint64_t *>(keys);
        else { sk = sort_keys(ctx, const_cast<uint64_t *>(keys), n, false, dlo, 8); own = true; }
    } else {
        sk = static_cast<uint64_t *>(ctx->alloc((n ? n : 1) * sizeof(uint64_t)));
        swap_words(ctx, keys, n, sk);
        own = true;
        sk = sort_keys(ctx, sk, n, true, dlo, 8);
    }
    if (unique_rows && n > 1 && !(canonical && col == 0 && arity == 2)) {
        uint64_t *u;
        const uint64_t un = unique_keys(ctx, sk, n, &u);
        if (own) ctx->free(sk);
        sk = u;
        own = true;
        n = un;
        J.n = un;
    }
    build_run_index(ctx, sk, n, J.ix);
    J.payload = Buf<uint32_t>(ctx, n ? n : 1);
    low_words(ctx, sk, n, J.payload.p);
    if (own) ctx->free(sk);
}

// Join step of a rule body with bounded memory.  A probe output of at most
// kChunkRows rows (default 2^30 - 1: 8 GiB of packed rows, one radix sort
// call) is emitted whole (a bag).  A larger one is emitted in tile
// ranges of at most kChunkRows rows; each range is sorted and deduplicated and
// merged into the result, which is then a sorted set.  Rule bodies only feed
// set operations (union, diff), so either form gives the same fixpoint, and
// duplicate-heavy joins (points-to hubs) no longer materialise their bag.
// XLOG_HIP_JOIN_CHUNK_ROWS overrides the chunk size (tests force multi-chunk
// folds with it, like the reference's XLOG_UNION_CHUNK_BYTES, relational.rs:36-42).
static uint64_t join_chunk_rows() {
    const char *e = getenv("XLOG_HIP_JOIN_CHUNK_ROWS");
    if (e && *e) {
        unsigned long long v = strtoull(e, nullptr, 10);
        if (v > 0) return v;
    }
    return (1ull << 30) - 1;
}
// XLOG_HIP_TRACE=1: one line on stderr per fixpoint iteration, per queue of
// iterations and per piece of a large join step (progress of long runs).
bool trace_on() {
    const char *e = getenv("XLOG_HIP_TRACE");
    return e && e[0] == '1';
}

// The emit side of a join step whose count pass has run (job.total known).
// digits: the sort's known varying digits (0: from the histograms).
uint64_t join_emit(Ctx *ctx, ProbeJob &job, const int oc[4], uint64_t **out, uint64_t max_rows, uint32_t digits) {
    const uint64_t kChunkRows = join_chunk_rows();
    const uint64_t total = job.total;
    *out = nullptr;
    if (total == 0) return 0;
    // the bag size is known before anything is materialised (the reference
    // refuses joins above its u32 row limit at the same point, relational.rs:4550-4555)
    XH_REQUIRE(max_rows == 0 || total <= max_rows, XLOG_HIP_CAPACITY_OVERFLOW,
               "Join produced " + std::to_string(total) + " rows which exceeds the row limit " +
                   std::to_string(max_rows));
    if (total <= kChunkRows) {
        uint64_t *o = static_cast<uint64_t *>(ctx->alloc(total * sizeof(uint64_t)));
        Owned go(ctx, o);
        probe_emit_range(ctx, job, 0, job.tiles, total, 2, oc, o, nullptr);
        *out = go.release();
        return total;
    }
    std::vector<uint64_t> off = probe_tile_offsets(ctx, job);
    Owned acc(ctx);
    uint64_t acc_n = 0;
    for (uint64_t t0 = 0; t0 < job.tiles;) {
        uint64_t t1 = t0 + 1;
        while (t1 < job.tiles && off[t1 + 1] - off[t0] <= kChunkRows) ++t1;
        const uint64_t m = off[t1] - off[t0];
        if (trace_on())
            fprintf(stderr, "[xlog_hip] join step of %llu rows: piece of %llu rows from tile %llu of %llu\n",
                    (unsigned long long)total, (unsigned long long)m, (unsigned long long)t0,
                    (unsigned long long)job.tiles);
        if (m) {
            uint64_t *b = static_cast<uint64_t *>(ctx->alloc(m * sizeof(uint64_t)));
            {
                Owned gb(ctx, b);
                probe_emit_range(ctx, job, t0, t1, m, 2, oc, b, nullptr);
                gb.release();
            }
            Owned srt(ctx, sort_keys(ctx, b, m, true, 0, 8, digits));  // consumes b
            uint64_t *u;
            uint64_t un = unique_keys(ctx, srt.p, m, &u);
            Owned gu(ctx, u);
            srt.reset();
            if (!acc.p) {
                acc.reset(gu.release());
                acc_n = un;
            } else {
                Owned mg(ctx, alloc_keys(ctx, acc_n + un));
                merge_sorted(ctx, acc.p, acc_n, u, un, mg.p);
                acc.reset();
                gu.reset();
                uint64_t *u2;
                uint64_t n2 = unique_keys(ctx, mg.p, acc_n + un, &u2);
                acc.reset(u2);
                acc_n = n2;
            }
        }
        t0 = t1;
    }
    *out = acc.release();
    return acc_n;
}
uint64_t join_step(Ctx *ctx, const uint64_t *probe, uint64_t n, int pcol, const JoinIndex &J, const int oc[4],
                   uint64_t **out, uint64_t max_rows, uint32_t digits) {
    ProbeJob job;
    job.probe = probe;
    job.n = n;
    job.pcol = pcol;
    job.ix = &J.ix;
    job.payload = J.payload.p;
    *out = nullptr;
    if (probe_prepare(ctx, job) == 0) return 0;
    return join_emit(ctx, job, oc, out, max_rows, digits);
}

// value-index of a relation column for the probe side: arity 1 stores c0 in
// the low word (v1), arity 2 stores c0 high (v0) and c1 low (v1)
static int probe_vidx(uint32_t arity, uint32_t c) { return arity == 1 ? 1 : (int)c; }

// Join of `l` against an index built over column rk of a relation of arity
// r_arity.  max_output > 0 keeps the first max_output rows of the output
// (row order: probe-row major).
static xlog_hip_rel *op_join_indexed(Ctx *ctx, const xlog_hip_rel *l, uint32_t lk, const JoinIndex &J, uint32_t r_arity,
                                     uint32_t rk, int type, const std::vector<int> *out_cols, uint64_t max_output = 0) {
    XH_REQUIRE(lk < l->arity, XLOG_HIP_INVALID_ARG, "join key column out of range");
    XH_REQUIRE(l->arity <= 2, XLOG_HIP_UNSUPPORTED, "join: input arity above 2 is not supported");
    const uint32_t r_arity_ = r_arity;
    const int pcol = probe_vidx(l->arity, lk);
    if (type == XLOG_HIP_JOIN_SEMI || type == XLOG_HIP_JOIN_ANTI) {
        Buf<uint8_t> flags(ctx, l->rows ? l->rows : 1);
        join_match_flags(ctx, l->w[0], l->rows, pcol, J.ix, type == XLOG_HIP_JOIN_SEMI, flags.p);
        return compact_rel(ctx, l, flags.p);
    }
    XH_REQUIRE(type == XLOG_HIP_JOIN_INNER, XLOG_HIP_INVALID_ARG, "unknown join type");
    // value index of every column of (left ++ right)
    std::vector<int> vmap;
    for (uint32_t c = 0; c < l->arity; ++c) vmap.push_back(probe_vidx(l->arity, c));
    for (uint32_t c = 0; c < r_arity_; ++c) vmap.push_back(c == rk ? 2 : 3);
    std::vector<int> sel;
    if (out_cols) {
        for (int c : *out_cols) {
            XH_REQUIRE(c >= 0 && c < (int)vmap.size(), XLOG_HIP_INVALID_ARG, "projection column out of range");
            sel.push_back(vmap[c]);
        }
    } else {
        sel = vmap;
    }
    XH_REQUIRE(!sel.empty() && sel.size() <= 4, XLOG_HIP_UNSUPPORTED, "join output arity must be 1..4");
    int oc[4] = {0, 0, 0, 0};
    for (size_t i = 0; i < sel.size(); ++i) oc[i] = sel[i];
    uint64_t *o0 = nullptr, *o1 = nullptr;
    uint64_t n = join_probe_general(ctx, l->w[0], l->rows, pcol, J.ix, J.payload.p, (int)sel.size(), oc, &o0, &o1);
    if (n == 0) return rel_new(ctx, (uint32_t)sel.size(), 0);
    if (max_output && n > max_output) n = max_output;
    return rel_adopt(ctx, (uint32_t)sel.size(), n, o0, o1, 0);
}

static xlog_hip_rel *op_join_keys(Ctx *ctx, const xlog_hip_rel *l, const xlog_hip_rel *r, const std::vector<int> &lk,
                                  const std::vector<int> &rk, int type);
static xlog_hip_rel *op_project(Ctx *ctx, const xlog_hip_rel *in, const std::vector<int> &cols);

static xlog_hip_rel *op_join(Ctx *ctx, const xlog_hip_rel *l, const xlog_hip_rel *r, uint32_t lk, uint32_t rk,
                             int type, const std::vector<int> *out_cols) {
    XH_REQUIRE(l && r, XLOG_HIP_INVALID_ARG, "join input is NULL");
    XH_REQUIRE(lk < l->arity && rk < r->arity, XLOG_HIP_INVALID_ARG, "join key column out of range");
    if (l->arity > 2 || r->arity > 2) {
        // wider rows: the keyed join with one key column, then the projection
        xlog_hip_rel *j = op_join_keys(ctx, l, r, {(int)lk}, {(int)rk}, type);
        if (!out_cols || type != XLOG_HIP_JOIN_INNER) return j;
        std::unique_ptr<xlog_hip_rel, void (*)(xlog_hip_rel *)> jg(j, rel_free);
        return op_project(ctx, j, *out_cols);
    }
    JoinIndex J;
    build_join_index(ctx, r->w[0], r->rows, r->arity, (int)rk, (r->flags & REL_CANONICAL) != 0, J);
    return op_join_indexed(ctx, l, lk, J, r->arity, rk, type, out_cols);
}

// ---------------------------------------------------------------------------
// Equi-join on lists of key columns, inputs of any arity (reference
// hash_join_v2 with key lists, relational.rs:2926-2992, whose keys are packed
// row-major and hashed by pack_and_hash_keys, pack.cu:144-214).
//
// Instead of hashing variable-length packed key bytes, every key column is
// folded into a dense u32 id: the first step keys each row by its first one or
// two key columns as one u64, later steps by (previous id << 32) | next key
// column; the id is the key's rank among the build side's sorted unique keys
// (a left key absent from the build side gets KEY_NONE, which no build id
// equals).  The equal-id join then runs on (id << 32) | row words through the
// single-key run index and the wave-cooperative probe, which emit
// (left row << 32) | right row in left-row-major, right-row order; a gather
// writes the left ++ right columns.
// ---------------------------------------------------------------------------
namespace {
constexpr uint32_t KEY_NONE = 0xFFFFFFFFu;

// u64 key of one folding step: (hi << 32) | column c1, hi = prev[i] when given,
// else column c0; c1 < 0 keys by hi alone
__global__ void k_fold_key(RelView in, const uint32_t *__restrict__ prev, int c0, int c1, uint64_t n,
                           uint64_t *__restrict__ out) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t hi = prev ? (uint64_t)prev[i] : (uint64_t)col_value(in, c0, i);
        out[i] = c1 < 0 ? hi : ((hi << 32) | col_value(in, c1, i));
    }
}
// rank of each key among the sorted unique keys u[0..nu), KEY_NONE when absent
__global__ void k_rank_ids(const uint64_t *__restrict__ keys, uint64_t n, const uint64_t *__restrict__ u, uint64_t nu,
                           uint32_t *__restrict__ ids) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t k = keys[i];
        uint64_t lo = 0, hi = nu;
        while (lo < hi) {
            const uint64_t mid = lo + ((hi - lo) >> 1);
            if (u[mid] < k) lo = mid + 1; else hi = mid;
        }
        ids[i] = (lo < nu && u[lo] == k) ? (uint32_t)lo : KEY_NONE;
    }
}
// (id << 32) | row index
__global__ void k_id_rows(const uint32_t *__restrict__ ids, uint64_t n, uint64_t *__restrict__ out) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = ((uint64_t)ids[i] << 32) | (uint32_t)i;
}
__global__ void k_found_flags(const uint32_t *__restrict__ ids, uint64_t n, int want, uint8_t *__restrict__ flags) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        flags[i] = (ids[i] != KEY_NONE) == (want != 0);
}
// output row r = left row (pairs[r] >> 32) ++ right row (low word)
__global__ void k_gather_pairs(RelView L, RelView R, const uint64_t *__restrict__ pairs, uint64_t n, RelOut out) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    const int arity = L.arity + R.arity;
    for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < n; r += stride) {
        const uint64_t pr = pairs[r];
        const uint64_t i = pr >> 32, j = (uint32_t)pr;
        uint32_t v[MAX_ARITY];
        for (int c = 0; c < L.arity; ++c) v[c] = col_value(L, c, i);
        for (int c = 0; c < R.arity; ++c) v[L.arity + c] = col_value(R, c, j);
        put_row(out, arity, v, r);
    }
}
// output row r = left row (w[r] >> 32) ++ the right row rebuilt from the
// left row's key value and the index payload (low word): the direct index
// over one key column of a right relation of at most two columns
__global__ void k_gather_left_payload(RelView L, int lk, int r_arity, int rk, const uint64_t *__restrict__ w,
                                      uint64_t n, RelOut out) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    const int arity = L.arity + r_arity;
    for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < n; r += stride) {
        const uint64_t x = w[r];
        const uint64_t i = x >> 32;
        uint32_t v[MAX_ARITY];
        for (int c = 0; c < L.arity; ++c) v[c] = col_value(L, c, i);
        const uint32_t key = col_value(L, lk, i);
        if (r_arity == 1) {
            v[L.arity] = key;
        } else {
            v[L.arity + rk] = key;
            v[L.arity + 1 - rk] = (uint32_t)x;
        }
        put_row(out, arity, v, r);
    }
}
// (column c << 32) | row index
__global__ void k_key_rows(RelView in, int c, uint64_t n, uint64_t *__restrict__ out) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = ((uint64_t)col_value(in, c, i) << 32) | (uint32_t)i;
}
}  // namespace

// The folding steps of a key list of nk columns: step 0 keys by columns
// (c[0], c[1]) as one u64 (c[0] alone when nk == 1), step s >= 1 by
// (id of step s - 1, c[s + 1]).
static size_t fold_steps(size_t nk) { return nk >= 2 ? nk - 1 : 1; }
static void fold_cols(const std::vector<int> &c, size_t step, int *c0, int *c1) {
    if (step == 0) {
        *c0 = c[0];
        *c1 = c.size() >= 2 ? c[1] : -1;
    } else {
        *c0 = -1;
        *c1 = c[step + 1];
    }
}

// The build side's fold over its key columns rk: every step's dictionary
// (sorted unique keys) and, with runs, the run index over (id << 32) | row
// (a stable sort, so a run lists its rows in input order).
static void fold_build(Ctx *ctx, const xlog_hip_rel *r, const std::vector<int> &rk, KeyFold &F, bool runs) {
    const uint64_t nr = r->rows;
    Buf<uint32_t> rid(ctx, nr);
    Buf<uint64_t> rkey(ctx, nr);
    for (size_t st = 0; st < fold_steps(rk.size()); ++st) {
        int c0, c1;
        fold_cols(rk, st, &c0, &c1);
        LAUNCH_1D(k_fold_key, nr, view_of(r), st == 0 ? nullptr : rid.p, c0, c1, nr, rkey.p);
        uint64_t *sorted = sort_keys(ctx, rkey.p, nr, false);
        uint64_t *u = nullptr;
        uint64_t nu = 0;
        try {
            nu = unique_keys(ctx, sorted, nr, &u);
        } catch (...) {
            ctx->free(sorted);
            throw;
        }
        ctx->free(sorted);
        Buf<uint64_t> d;
        d.ctx = ctx;
        d.p = u;
        d.n = nu;
        F.dict.push_back(std::move(d));
        F.dict_n.push_back(nu);
        LAUNCH_1D(k_rank_ids, nr, rkey.p, nr, u, nu, rid.p);
    }
    if (!runs) return;
    Buf<uint64_t> rp(ctx, nr);
    LAUNCH_1D(k_id_rows, nr, rid.p, nr, rp.p);
    rid = Buf<uint32_t>();
    rkey = Buf<uint64_t>();
    build_join_index(ctx, rp.p, nr, 2, 0, false, F.J);
}

// The probe side's ids in the build side's dictionaries (KEY_NONE for a key
// no build row has: it stays KEY_NONE through later steps, since every
// dictionary key of a later step has a build id, below KEY_NONE, in its high
// word).
static void fold_probe(Ctx *ctx, const xlog_hip_rel *l, const std::vector<int> &lk, const KeyFold &F,
                       Buf<uint32_t> &lid, Buf<uint64_t> &lkey) {
    const uint64_t nl = l->rows;
    for (size_t st = 0; st < fold_steps(lk.size()); ++st) {
        int c0, c1;
        fold_cols(lk, st, &c0, &c1);
        LAUNCH_1D(k_fold_key, nl, view_of(l), st == 0 ? nullptr : lid.p, c0, c1, nl, lkey.p);
        LAUNCH_1D(k_rank_ids, nl, lkey.p, nl, F.dict[st].p, F.dict_n[st], lid.p);
    }
}

// The join of non-empty inputs against the fold of r: INNER rows left ++
// right in left-row-major, right-row order (the first max_output when set),
// SEMI / ANTI the left rows with / without a match in input order.
static xlog_hip_rel *keyed_join_probe(Ctx *ctx, const xlog_hip_rel *l, const xlog_hip_rel *r,
                                      const std::vector<int> &lk, const KeyFold &F, int type, uint64_t max_output) {
    const uint64_t nl = l->rows;
    const uint32_t arity = l->arity + r->arity;
    Buf<uint32_t> lid(ctx, nl);
    Buf<uint64_t> lkey(ctx, nl);
    fold_probe(ctx, l, lk, F, lid, lkey);
    if (type != XLOG_HIP_JOIN_INNER) {
        Buf<uint8_t> flags(ctx, nl);
        LAUNCH_1D(k_found_flags, nl, lid.p, nl, type == XLOG_HIP_JOIN_SEMI ? 1 : 0, flags.p);
        xlog_hip_rel *o = compact_rel(ctx, l, flags.p);
        if (l->flags & REL_CANONICAL) o->flags = REL_CANONICAL;  // a subset of a sorted set is one
        return o;
    }
    // (id << 32) | row on the probe side (the left keys are no longer needed)
    LAUNCH_1D(k_id_rows, nl, lid.p, nl, lkey.p);
    lid = Buf<uint32_t>();
    const int oc[4] = {1, 3, 0, 0};  // (left row << 32) | right row
    uint64_t *pairs = nullptr;
    uint64_t n = join_probe_general(ctx, lkey.p, nl, 0, F.J.ix, F.J.payload.p, 2, oc, &pairs, nullptr);
    if (n == 0) return rel_new(ctx, arity, 0);
    Buf<uint64_t> pb;
    pb.ctx = ctx;
    pb.p = pairs;
    if (max_output && n > max_output) n = max_output;
    std::unique_ptr<xlog_hip_rel, void (*)(xlog_hip_rel *)> o(rel_new(ctx, arity, n), rel_free);
    o->rows = n;
    LAUNCH_1D(k_gather_pairs, n, view_of(l), view_of(r), pairs, n, out_of(o.get()));
    return o.release();
}

// The join of l (any arity) against the direct index over column rk of a
// relation of r_arity <= 2 columns: probe words (key << 32) | left row, the
// right row rebuilt from the key and the payload.
static xlog_hip_rel *direct_join_wide_left(Ctx *ctx, const xlog_hip_rel *l, uint32_t lk, const JoinIndex &J,
                                           uint32_t r_arity, uint32_t rk, int type, uint64_t max_output) {
    const uint64_t nl = l->rows;
    Buf<uint64_t> probe(ctx, nl);
    LAUNCH_1D(k_key_rows, nl, view_of(l), (int)lk, nl, probe.p);
    if (type != XLOG_HIP_JOIN_INNER) {
        Buf<uint8_t> flags(ctx, nl);
        join_match_flags(ctx, probe.p, nl, 0, J.ix, type == XLOG_HIP_JOIN_SEMI, flags.p);
        xlog_hip_rel *o = compact_rel(ctx, l, flags.p);
        if (l->flags & REL_CANONICAL) o->flags = REL_CANONICAL;
        return o;
    }
    const uint32_t arity = l->arity + r_arity;
    XH_REQUIRE(arity <= MAX_ARITY, XLOG_HIP_UNSUPPORTED, "join: output arity (left ++ right) above 8");
    const int oc[4] = {1, 3, 0, 0};  // (left row << 32) | payload
    uint64_t *w = nullptr;
    uint64_t n = join_probe_general(ctx, probe.p, nl, 0, J.ix, J.payload.p, 2, oc, &w, nullptr);
    if (n == 0) return rel_new(ctx, arity, 0);
    Buf<uint64_t> wb;
    wb.ctx = ctx;
    wb.p = w;
    if (max_output && n > max_output) n = max_output;
    std::unique_ptr<xlog_hip_rel, void (*)(xlog_hip_rel *)> o(rel_new(ctx, arity, n), rel_free);
    o->rows = n;
    LAUNCH_1D(k_gather_left_payload, n, view_of(l), (int)lk, (int)r_arity, (int)rk, w, n, out_of(o.get()));
    return o.release();
}

static void check_key_lists(const xlog_hip_rel *l, const xlog_hip_rel *r, const std::vector<int> &lk,
                            const std::vector<int> &rk, int type) {
    XH_REQUIRE(l && r, XLOG_HIP_INVALID_ARG, "join input is NULL");
    XH_REQUIRE(!lk.empty() && lk.size() == rk.size(), XLOG_HIP_INVALID_ARG,
               "join: key column lists must be non-empty and of equal length");
    for (size_t t = 0; t < lk.size(); ++t)
        XH_REQUIRE(lk[t] >= 0 && lk[t] < (int)l->arity && rk[t] >= 0 && rk[t] < (int)r->arity, XLOG_HIP_INVALID_ARG,
                   "join key column out of range");
    XH_REQUIRE(type == XLOG_HIP_JOIN_INNER || type == XLOG_HIP_JOIN_SEMI || type == XLOG_HIP_JOIN_ANTI,
               XLOG_HIP_INVALID_ARG, "unknown join type");
    XH_REQUIRE(type != XLOG_HIP_JOIN_INNER || l->arity + r->arity <= MAX_ARITY, XLOG_HIP_UNSUPPORTED,
               "join: output arity (left ++ right) above 8");
    XH_REQUIRE(l->rows < KEY_NONE && r->rows < KEY_NONE, XLOG_HIP_CAPACITY_OVERFLOW,
               "join: more than 2^32 - 2 rows on one side");
}
// The result of a join with an empty side (reference relational.rs:3920-3940).
static xlog_hip_rel *empty_side_join(Ctx *ctx, const xlog_hip_rel *l, const xlog_hip_rel *r, int type) {
    if (type == XLOG_HIP_JOIN_ANTI) return rel_clone(ctx, l);
    return rel_new(ctx, type == XLOG_HIP_JOIN_INNER ? l->arity + r->arity : l->arity, 0);
}

static xlog_hip_rel *op_join_keys(Ctx *ctx, const xlog_hip_rel *l, const xlog_hip_rel *r, const std::vector<int> &lk,
                                  const std::vector<int> &rk, int type) {
    check_key_lists(l, r, lk, rk, type);
    if (l->rows == 0 || r->rows == 0) return empty_side_join(ctx, l, r, type);
    KeyFold F;
    fold_build(ctx, r, rk, F, type == XLOG_HIP_JOIN_INNER);
    return keyed_join_probe(ctx, l, r, lk, F, type, 0);
}

static bool column_sorted(Ctx *ctx, const xlog_hip_rel *rel, uint32_t col) {
    if (rel->rows < 2) return true;
    Buf<uint32_t> flag(ctx, 1);
    fill_u32(ctx, flag.p, 0u, 1);
    LAUNCH_1D(k_col_unsorted, rel->rows, view_of(rel), (int)col, rel->rows, flag.p);
    uint32_t h = 0;
    XH_CHECK_HIP(hipMemcpyAsync(&h, flag.p, 4, hipMemcpyDeviceToHost, ctx->stream));
    ctx->sync();
    return h == 0;
}

// Sort-merge inner join (reference sort_merge_join_v2_inner_u32_1key,
// relational.rs:3401-3571): output columns left ++ right like the hash join.
// The reference requires both sides sorted ascending on their key and at
// most 4,000,000 row pairs; here a side whose key column is not sorted is
// sorted (stably, key word only) and there is no pair cap.  The right side's
// runs of equal keys are matched to the left rows along the merge path
// (smj_lookup); the matches are expanded by the probe's count / emit.  Rows
// come out left-row-major (in key order), right rows of a run in input order.
static xlog_hip_rel *op_sort_merge_join(Ctx *ctx, const xlog_hip_rel *l, const xlog_hip_rel *r, uint32_t lk,
                                        uint32_t rk) {
    XH_REQUIRE(l && r, XLOG_HIP_INVALID_ARG, "join input is NULL");
    XH_REQUIRE(lk < l->arity && rk < r->arity, XLOG_HIP_INVALID_ARG, "join key column out of range");
    XH_REQUIRE(l->arity <= 2 && r->arity <= 2, XLOG_HIP_UNSUPPORTED, "join: input arity above 2 is not supported");
    const uint32_t arity = l->arity + r->arity;
    if (l->rows == 0 || r->rows == 0) return rel_new(ctx, arity, 0);
    // right side as (key << 32) | other column, ordered by key
    const uint64_t nr = r->rows;
    // every buffer of this operator is owned by a Buf, so an error on the way frees them
    auto adopt = [&](uint64_t *q, uint64_t count) {
        Buf<uint64_t> b;
        b.ctx = ctx;
        b.p = q;
        b.n = count;
        return b;
    };
    Buf<uint64_t> rs(ctx, nr);
    if (r->arity == 2 && rk == 0) copy_d2d(ctx, rs.p, r->w[0], nr);
    else swap_words(ctx, r->w[0], nr, rs.p);  // arity 1 keeps c0 in the low word
    if (!column_sorted(ctx, r, rk)) rs = adopt(sort_keys(ctx, rs.p, nr, false, 4, 8), nr);
    JoinIndex J;  // runs and payload only; the sort-merge lookup needs no hash table
    J.n = nr;
    Buf<uint32_t> run_key(ctx, nr);
    Buf<uint64_t> run_start(ctx, nr + 1);
    {
        Buf<uint64_t> cnt(ctx, 1);
        select_runs(ctx, rs.p, nr, run_key.p, run_start.p, cnt.p);
        J.ix.nruns = read_count(ctx, cnt.p);
    }
    fill_u64(ctx, run_start.p + J.ix.nruns, nr, 1);  // run_start[nruns] = end
    J.payload = Buf<uint32_t>(ctx, nr);
    low_words(ctx, rs.p, nr, J.payload.p);
    rs = Buf<uint64_t>();
    // left side ordered by its key column (stable: key digits only)
    const int pcol = probe_vidx(l->arity, lk);
    Buf<uint64_t> ls;
    const uint64_t *probe = l->w[0];
    if (!column_sorted(ctx, l, lk)) {
        ls = adopt(sort_keys(ctx, const_cast<uint64_t *>(l->w[0]), l->rows, false, pcol ? 0 : 4, pcol ? 4 : 8),
                   l->rows);
        probe = ls.p;
    }
    Buf<uint64_t> pre_start(ctx, l->rows);
    Buf<uint32_t> pre_cnt(ctx, l->rows);
    {
        Prof prof(ctx, XLOG_HIP_KERNEL_MERGE, 8.0 * (double)l->rows + 4.0 * (double)J.ix.nruns);
        smj_lookup(ctx, probe, l->rows, pcol, run_key.p, run_start.p, J.ix.nruns, pre_start.p, pre_cnt.p);
    }
    std::vector<int> vmap;  // value index of every output column (left ++ right)
    for (uint32_t c = 0; c < l->arity; ++c) vmap.push_back(probe_vidx(l->arity, c));
    for (uint32_t c = 0; c < r->arity; ++c) vmap.push_back(c == rk ? 2 : 3);
    int oc[4] = {0, 0, 0, 0};
    for (size_t i = 0; i < vmap.size(); ++i) oc[i] = vmap[i];
    ProbeJob job;
    job.probe = probe;
    job.n = l->rows;
    job.pcol = pcol;
    job.ix = &J.ix;
    job.payload = J.payload.p;
    job.pre_start = pre_start.p;
    job.pre_cnt = pre_cnt.p;
    const uint64_t total = probe_prepare(ctx, job);
    if (total == 0) return rel_new(ctx, arity, 0);
    Buf<uint64_t> o0(ctx, total), o1(ctx, arity > 2 ? total : 0);
    probe_emit_range(ctx, job, 0, job.tiles, total, (int)arity, oc, o0.p, o1.p);
    return rel_adopt(ctx, arity, total, o0.release(), o1.release(), 0);
}

// Nested-loop inner join (reference nested_loop_join_v2_inner_u32_1key,
// relational.rs:3041-3255): same output columns as the inner hash join, rows
// in left-row-major, right-row order; refused above rows_l * rows_r =
// 4,000,000 like the reference (NESTED_LOOP_TOTAL_THRESHOLD, provider/mod.rs:1030).
static xlog_hip_rel *op_nested_loop_join(Ctx *ctx, const xlog_hip_rel *l, const xlog_hip_rel *r, uint32_t lk,
                                         uint32_t rk) {
    XH_REQUIRE(l && r, XLOG_HIP_INVALID_ARG, "join input is NULL");
    XH_REQUIRE(lk < l->arity && rk < r->arity, XLOG_HIP_INVALID_ARG, "join key column out of range");
    XH_REQUIRE(l->arity <= 2 && r->arity <= 2, XLOG_HIP_UNSUPPORTED, "join: input arity above 2 is not supported");
    const uint32_t arity = l->arity + r->arity;
    if (l->rows == 0 || r->rows == 0) return rel_new(ctx, arity, 0);
    XH_REQUIRE(l->rows <= 4000000ull / r->rows, XLOG_HIP_CAPACITY_OVERFLOW,
               "nested loop join: rows_l * rows_r exceeds 4000000");
    uint64_t *o0, *o1;
    const uint64_t n = nested_loop_join(ctx, l->w[0], l->rows, (int)l->arity, (int)lk, r->w[0], r->rows,
                                        (int)r->arity, (int)rk, &o0, &o1);
    if (n == 0) return rel_new(ctx, arity, 0);
    return rel_adopt(ctx, arity, n, o0, o1, 0);
}

// Dedup of input ordered on the key columns (reference dedup_sorted,
// relational.rs:288-420): full-row keys of arity > 1 take the full-row dedup;
// otherwise the first row of every run of adjacent rows equal on the key
// columns is kept, in input order, without sorting.
static xlog_hip_rel *op_dedup_sorted(Ctx *ctx, const xlog_hip_rel *in, const std::vector<int> &cols) {
    XH_REQUIRE(!cols.empty(), XLOG_HIP_INVALID_ARG, "dedup needs at least one key column");
    if (in->arity > 1 && is_full_key(in, cols)) return op_dedup_full(ctx, in);
    if (in->rows <= 1) return rel_clone(ctx, in);
    std::vector<int> keys;  // distinct key columns (at most the arity, <= 4)
    for (int c : cols)
        if (std::find(keys.begin(), keys.end(), c) == keys.end()) keys.push_back(c);
    Buf<uint8_t> flags(ctx, in->rows);
    ProjSpec ks{(int)in->arity, (int)keys.size(), {0, 0, 0, 0, 0, 0, 0, 0}};
    for (int j = 0; j < ks.out_arity; ++j) ks.cols[j] = keys[j];
    LAUNCH_1D(k_group_flags, in->rows, view_of(in), ks, in->rows, flags.p);
    xlog_hip_rel *r = compact_rel(ctx, in, flags.p);
    if (in->flags & REL_CANONICAL) r->flags = REL_CANONICAL;  // a subset of a sorted set is one
    return r;
}

// One factorized TC delta step (reference fj_delta_novel_u32_recorded,
// crates/xlog-cuda/src/provider/fj_delta.rs:117-490): the set
//   { head(carry, value) : delta(carry, key), edge(key, value), head not in full }
// with the column roles of `cols`, output in full's column order (r_carry,
// r_value), canonical.  Every id must be below `domain` <= 2^16.
static xlog_hip_rel *op_fj_delta(Ctx *ctx, const xlog_hip_rel *delta, const xlog_hip_rel *edge,
                                 const xlog_hip_rel *full, const xlog_hip_fj_delta_cols &c, uint32_t domain) {
    XH_REQUIRE(delta && edge && full, XLOG_HIP_INVALID_ARG, "fj delta: input is NULL");
    XH_REQUIRE(delta->arity == 2 && edge->arity == 2 && full->arity == 2, XLOG_HIP_INVALID_ARG,
               "fj delta: delta, edge and full must be arity-2");
    auto roles_ok = [](uint32_t a, uint32_t b) { return a < 2 && b < 2 && a != b; };
    XH_REQUIRE(roles_ok(c.delta_carry, c.delta_key) && roles_ok(c.r_carry, c.r_value), XLOG_HIP_INVALID_ARG,
               "fj delta: invalid column roles (arity-2 indices, pairwise distinct)");
    XH_REQUIRE(domain > 0 && domain <= (1u << 16), XLOG_HIP_INVALID_ARG, "fj delta: domain outside (0, 2^16]");
    if (delta->rows == 0 || edge->rows == 0) {
        xlog_hip_rel *e = rel_new(ctx, 2, 0);
        e->flags = REL_CANONICAL;
        return e;
    }
    {  // every id below the domain (checked before any bitmap is touched)
        Buf<unsigned int> mx(ctx, 1);
        fill_u32(ctx, mx.p, 0u, 1);
        const xlog_hip_rel *rs[3] = {delta, edge, full};
        for (const xlog_hip_rel *r : rs)
            if (r->rows) MAX_LAUNCH_1D(k_max_u32_of_packed, r->rows, r->w[0], r->rows, mx.p);
        uint32_t h = 0;
        XH_CHECK_HIP(hipMemcpyAsync(&h, mx.p, 4, hipMemcpyDeviceToHost, ctx->stream));
        ctx->sync();
        XH_REQUIRE(h < domain, XLOG_HIP_INVALID_ARG,
                   "fj delta: id " + std::to_string(h) + " outside the domain " + std::to_string(domain));
    }
    Canon ce;  // edge as sorted unique (key << 32) | value
    canonical_keys(ctx, edge, ce);
    uint64_t *o = nullptr;
    const uint64_t n = fj_delta_step(ctx, delta->w[0], delta->rows, c.delta_carry == 0 ? 1 : 0, ce.k, ce.n,
                                     full->w[0], full->rows, c.r_carry == 0 ? 1 : 0, domain, &o);
    if (n == 0) {
        xlog_hip_rel *e = rel_new(ctx, 2, 0);
        e->flags = REL_CANONICAL;
        return e;
    }
    if (c.r_carry == 1) {  // head column order (value, carry): swap and re-sort
        uint64_t *sw = static_cast<uint64_t *>(ctx->alloc(n * sizeof(uint64_t)));
        swap_words(ctx, o, n, sw);
        ctx->free(o);
        o = sort_keys(ctx, sw, n, true);  // consumes sw
    }
    return rel_adopt(ctx, 2, n, o, nullptr, REL_CANONICAL);
}

// One sparse factorized delta step (reference fj_delta_sparse_novel_u32_recorded,
// crates/xlog-cuda/src/provider/fj_delta_sparse.rs:66-490): the set
//   { head(carry, value) : delta(carry, key), edge(key, value), head not in full }
// with no domain bound, over a device hash set filled with `full`.  The
// table is sized 2 x (|full| + candidates), the candidate count coming from
// the probe's count pass (an upper bound of the distinct candidates, which the
// reference estimates with a bitmap).  A table above max_table_bytes (when
// non-zero) declines, like the reference's Ok(None): *declined is set and no
// relation is returned.  The output is canonical in full's column order.
static xlog_hip_rel *op_fj_delta_sparse(Ctx *ctx, const xlog_hip_rel *delta, const xlog_hip_rel *edge,
                                        const xlog_hip_rel *full, const xlog_hip_fj_delta_cols &c,
                                        uint64_t max_table_bytes, bool *declined) {
    *declined = false;
    XH_REQUIRE(delta && edge && full, XLOG_HIP_INVALID_ARG, "fj delta sparse: input is NULL");
    XH_REQUIRE(delta->arity == 2 && edge->arity == 2 && full->arity == 2, XLOG_HIP_INVALID_ARG,
               "fj delta sparse: delta, edge and full must be arity-2");
    auto roles_ok = [](uint32_t a, uint32_t b) { return a < 2 && b < 2 && a != b; };
    XH_REQUIRE(roles_ok(c.delta_carry, c.delta_key) && roles_ok(c.r_carry, c.r_value), XLOG_HIP_INVALID_ARG,
               "fj delta sparse: invalid column roles (arity-2 indices, pairwise distinct)");
    auto empty = [&]() {
        xlog_hip_rel *e = rel_new(ctx, 2, 0);
        e->flags = REL_CANONICAL;
        return e;
    };
    if (delta->rows == 0 || edge->rows == 0) return empty();
    Canon ce;  // edge as sorted unique (key << 32) | value: runs of values per key
    canonical_keys(ctx, edge, ce);
    JoinIndex J;
    build_join_index(ctx, ce.k, ce.n, 2, 0, true, J);
    ProbeJob job;  // count pass only: the number of candidate tuples
    job.probe = delta->w[0];
    job.n = delta->rows;
    job.pcol = c.delta_key == 0 ? 0 : 1;
    job.ix = &J.ix;
    job.payload = J.payload.p;
    job.record_lookups = false;
    const uint64_t cand = probe_prepare(ctx, job);
    if (cand == 0) return empty();
    uint64_t slots = 1ull << 16;
    while (slots < 2 * (full->rows + cand)) slots <<= 1;
    if (max_table_bytes && slots * sizeof(uint64_t) > max_table_bytes) {
        *declined = true;
        return nullptr;
    }
    HashSet h;
    hs_init(ctx, h, slots);
    hs_insert_all(ctx, h, full->w[0], full->rows);
    h.size = full->rows;
    // the novel tuples number at most `cand`, so a limit of cand + 1 is never reached
    Buf<uint64_t> novel(ctx, cand + 1 + HS_APPEND_SLACK);
    hs_join_insert(ctx, h, delta->w[0], delta->rows, c.delta_key == 0 ? 1 : 0, c.r_carry == 0 ? 1 : 0, J.ix,
                   J.payload.p, novel.p, cand + 1);
    ctx->read_scalars(h.flags.p + 1, 2);
    XH_REQUIRE(ctx->host_scalars[0] == 0, XLOG_HIP_DEVICE_ERROR, "fj delta sparse: table overflow");
    const uint64_t n = ctx->host_scalars[1];
    if (n == 0) return empty();
    h = HashSet();
    uint64_t *s = sort_keys(ctx, novel.p, n, false);
    return rel_adopt(ctx, 2, n, s, nullptr, REL_CANONICAL);
}

// Set of the projected join, canonical: dedup_full_row(project(join(l, r))).
// When the output is (left column, right non-key column) the join is emitted
// already ordered: the probe side is first sorted by its output column (key
// word only) and the build runs are kept sorted by their payload, so each probe
// row's outputs are ascending and rows come in output-column order.  Only
// groups of probe rows that share the output column interleave; those runs
// are sorted in place (LDS bitonic sort per run), then one unique pass.  This
// replaces the radix sort of the whole join output.  Other shapes take the
// join -> sort -> unique path.
void left_keys(Ctx *ctx, const uint64_t *l, uint64_t n, int arity, int oc0, int jk, uint64_t *out);
void group_rows_async(Ctx *ctx, const uint64_t *k, uint64_t n, int32_t *gsel, uint64_t *mkeys, uint64_t *mpos,
                      uint64_t *hkeys, uint64_t *hpos, uint64_t *d_nm, uint64_t *d_nh);
void group_segments(Ctx *ctx, const uint64_t *sorted, uint64_t n, const uint64_t *head_keys, uint64_t nh,
                    uint64_t *seg, const uint64_t *d_n);
void sort_segments_async(Ctx *ctx, uint64_t *data, uint64_t n, const uint64_t *heads, uint64_t nh, uint64_t *seg,
                         unsigned long long *d_max);
void sort_segments_long(Ctx *ctx, uint64_t *data, const uint64_t *seg, uint64_t nh, uint64_t max_len);

namespace {
__global__ void k_gather_u64(const uint64_t *a, const uint64_t *b, uint64_t *out) {
    out[0] = *a;
    out[1] = *b;
}
}  // namespace

static xlog_hip_rel *op_join_project_dedup(Ctx *ctx, const xlog_hip_rel *l, const xlog_hip_rel *r, uint32_t lk,
                                           uint32_t rk, const std::vector<int> &out_cols) {
    XH_REQUIRE(l && r, XLOG_HIP_INVALID_ARG, "join input is NULL");
    XH_REQUIRE(lk < l->arity && rk < r->arity, XLOG_HIP_INVALID_ARG, "join key column out of range");
    const bool ordered = l->arity <= 2 && r->arity == 2 && out_cols.size() == 2 && out_cols[0] >= 0 &&
                         out_cols[0] < (int)l->arity && out_cols[1] == (int)l->arity + (1 - (int)rk);
    if (!ordered) {
        xlog_hip_rel *j = op_join(ctx, l, r, lk, rk, XLOG_HIP_JOIN_INNER, &out_cols);
        xlog_hip_rel *d = nullptr;
        try {
            d = op_dedup_full(ctx, j);
        } catch (...) {
            rel_free(j);
            throw;
        }
        rel_free(j);
        return d;
    }
    const uint64_t n = l->rows, nr = r->rows;
    auto empty = [&]() {
        xlog_hip_rel *e = rel_new(ctx, 2, 0);
        e->flags = REL_CANONICAL;
        return e;
    };
    if (n == 0 || nr == 0) return empty();
    // The host waits three times: for the build side's and the groups' sizes,
    // for the side probe's size (while the device runs the main count pass),
    // and for the output size (plus the sorts' histogram read-backs, which
    // their first digit pass overlaps).
    // 1. probe keys (out column << 32 | join key), ordered by the out column
    Buf<uint64_t> lk_buf;  // owns the sorted probe keys
    lk_buf.ctx = ctx;
    //    (or by the whole key, when the segment route of many keys does that in fewer passes)
    bool whole = false;
    if (l->arity == 2 && out_cols[0] == 0 && lk == 1) {
        // the rows are already (out column << 32 | join key): the sort reads them directly
        lk_buf.p = sort_keys(ctx, l->w[0], n, false, 4, 8, 0, &whole);
    } else {
        lk_buf.p = static_cast<uint64_t *>(ctx->alloc(n * sizeof(uint64_t)));
        left_keys(ctx, l->w[0], n, (int)l->arity, out_cols[0], (int)lk, lk_buf.p);
        lk_buf.p = sort_keys(ctx, lk_buf.p, n, true, 4, 8, 0, &whole);
    }
    const uint64_t *lkeys = lk_buf.p;
    // 2. build rows as (key << 32 | payload), sorted and unique, so that a probe
    //    row alone with its out column emits sorted, unique outputs
    //    (the key word's radix passes, then each run of equal keys sorted by
    //    payload in one pass; a run of more than 256 rows makes the build
    //    rows take the payload's radix passes too, after the first read-back)
    Buf<uint64_t> cnt(ctx, 5);  // unique build rows, runs, group members, groups, long run
    Buf<uint64_t> kw_buf, sk_buf;
    kw_buf.ctx = sk_buf.ctx = ctx;
    const uint64_t *sk;
    const bool canon = rk == 0 && (r->flags & REL_CANONICAL) != 0;
    if (canon) {
        sk = r->w[0];
        fill_u64(ctx, cnt.p + 4, 0ull, 1);
    } else {
        if (rk == 0) {
            kw_buf.p = sort_keys(ctx, r->w[0], nr, false, 4, 8, 0, &whole);
        } else {
            kw_buf.p = static_cast<uint64_t *>(ctx->alloc(nr * sizeof(uint64_t)));
            swap_words(ctx, r->w[0], nr, kw_buf.p);
            kw_buf.p = sort_keys(ctx, kw_buf.p, nr, true, 4, 8, 0, &whole);
        }
        if (whole) {  // the segment route ordered the build rows by the whole key
            fill_u64(ctx, cnt.p + 4, 0ull, 1);
            sk = kw_buf.p;
        } else {
            sk_buf = Buf<uint64_t>(ctx, nr);
            sort_short_runs(ctx, kw_buf.p, nr, sk_buf.p, cnt.p + 4);
            sk = sk_buf.p;
        }
    }
    Buf<uint64_t> ub;
    JoinIndex J;
    J.payload = Buf<uint32_t>(ctx, nr);
    const uint64_t *bk = sk, *d_un = nullptr;
    if (!canon && nr > 1) {
        ub = Buf<uint64_t>(ctx, nr);
        select_unique_low(ctx, sk, nr, ub.p, J.payload.p, cnt.p);  // the payloads come with the unique rows
        bk = ub.p;
        d_un = cnt.p;
    } else {
        low_words(ctx, bk, nr, J.payload.p);
    }
    RunScratch rs;
    build_run_index_async(ctx, bk, nr, d_un, rs, cnt.p + 1);
    // 3. probe rows sharing their out column (groups) can emit the same
    //    output twice and interleave: their outputs are produced on the side
    //    (probe, sort inside each group, unique) and copied into place by the
    //    main emit through the group selector
    Buf<int32_t> gsel(ctx, n);
    Buf<uint64_t> mkeys(ctx, n), mpos(ctx, n), hkeys(ctx, n), hpos(ctx, n);
    group_rows_async(ctx, lkeys, n, gsel.p, mkeys.p, mpos.p, hkeys.p, hpos.p, cnt.p + 2, cnt.p + 3);
    ctx->read_scalars(cnt.p, 5);
    uint64_t un = d_un ? ctx->host_scalars[0] : nr, nruns = ctx->host_scalars[1];
    const uint64_t nm = ctx->host_scalars[2], nh = ctx->host_scalars[3];
    if (ctx->host_scalars[4]) {  // a long run: the full sort of the build rows
        sk_buf = Buf<uint64_t>();
        sk_buf.ctx = ctx;
        sk_buf.p = sort_keys(ctx, kw_buf.p, nr, false, 0, 8);
        select_unique_low(ctx, sk_buf.p, nr, ub.p, J.payload.p, cnt.p);
        build_run_index_async(ctx, ub.p, nr, cnt.p, rs, cnt.p + 1);
        ctx->read_scalars(cnt.p, 2);
        un = ctx->host_scalars[0];
        nruns = ctx->host_scalars[1];
    }
    kw_buf = Buf<uint64_t>();
    J.n = un;
    build_run_index_finish(ctx, rs, nruns, un, J.ix);
    sk_buf = Buf<uint64_t>();
    ub = Buf<uint64_t>();
    mpos = Buf<uint64_t>();
    // 4. the side probe's count, then the main count pass (group heads count
    //    zero until their groups are known); the side total comes back while
    //    the main count runs
    const int oc[4] = {0, 3, 0, 0};  // v0 = out column (probe high word), v3 = payload
    ProbeJob side;
    if (nm) {
        side.probe = mkeys.p;
        side.n = nm;
        side.pcol = 1;
        side.ix = &J.ix;
        side.payload = J.payload.p;
        probe_count_only(ctx, side);
        probe_scan_async(ctx, side);
        XH_CHECK_HIP(hipMemcpyAsync(ctx->host_scalars, side.toff.p + side.tiles, sizeof(uint64_t),
                                    hipMemcpyDeviceToHost, ctx->stream));
        XH_CHECK_HIP(hipEventRecord(ctx->ev_read, ctx->stream));
    }
    ProbeJob job;
    job.probe = lkeys;
    job.n = n;
    job.pcol = 1;
    job.ix = &J.ix;
    job.payload = J.payload.p;
    if (nm) job.gsel = gsel.p;  // gseg unset: heads deferred
    probe_count_only(ctx, job);
    // 5. group outputs: emit, sort inside each group, unique; each head then
    //    gets its group's unique words and count
    Buf<uint64_t> gseg, bag, seg, u2, nu2(ctx, 1);
    Buf<unsigned long long> mx(ctx, 1);
    uint64_t m2 = 0;
    if (nm) {
        ctx->wait_event(ctx->ev_read);
        m2 = ctx->host_scalars[0];
        probe_finish(side, nm, m2);
        gseg = Buf<uint64_t>(ctx, 2 * nh);
        if (m2) {
            bag = Buf<uint64_t>(ctx, m2);
            probe_emit_range(ctx, side, 0, side.tiles, m2, 2, oc, bag.p, nullptr);
            seg = Buf<uint64_t>(ctx, 2 * nh);
            sort_segments_async(ctx, bag.p, m2, hkeys.p, nh, seg.p, mx.p);
            u2 = Buf<uint64_t>(ctx, m2);
            select_unique(ctx, bag.p, m2, u2.p, nu2.p);
            group_segments(ctx, u2.p, m2, hkeys.p, nh, gseg.p, nu2.p);
        } else {
            fill_u64(ctx, gseg.p, 0ull, 2 * nh);
        }
        probe_group_fixup(ctx, job, hpos.p, gseg.p, nh);
    }
    if (!nm || !m2) fill_u64(ctx, reinterpret_cast<uint64_t *>(mx.p), 0ull, 1);
    probe_scan_async(ctx, job);
    Buf<uint64_t> g2(ctx, 2);
    hipLaunchKernelGGL(k_gather_u64, dim3(1), dim3(1), 0, ctx->stream, job.toff.p + job.tiles,
                       reinterpret_cast<const uint64_t *>(mx.p), g2.p);
    XH_CHECK_HIP(hipGetLastError());
    ctx->read_scalars(g2.p, 2);
    uint64_t total = ctx->host_scalars[0];
    const uint64_t max_len = ctx->host_scalars[1];
    if (max_len > (uint64_t)WAVE) {
        // rare: a group with more than 64 outputs needs the block / radix
        // segment sorts; its unique words and the counts are then redone
        sort_segments_long(ctx, bag.p, seg.p, nh, max_len);
        select_unique(ctx, bag.p, m2, u2.p, nu2.p);
        group_segments(ctx, u2.p, m2, hkeys.p, nh, gseg.p, nu2.p);
        probe_count_only(ctx, job);
        probe_group_fixup(ctx, job, hpos.p, gseg.p, nh);
        probe_scan_async(ctx, job);
        ctx->read_scalars(job.toff.p + job.tiles, 1);
        total = ctx->host_scalars[0];
    }
    probe_finish(job, n, total);
    if (nm) {
        job.gseg = gseg.p;
        job.gsrc = u2.p;
    }
    if (!total) return empty();
    uint64_t *o = static_cast<uint64_t *>(ctx->alloc(total * sizeof(uint64_t)));
    try {
        probe_emit_range(ctx, job, 0, job.tiles, total, 2, oc, o, nullptr);
    } catch (...) {
        ctx->free(o);
        throw;
    }
    return rel_adopt(ctx, 2, total, o, nullptr, REL_CANONICAL);
}

static xlog_hip_rel *op_project(Ctx *ctx, const xlog_hip_rel *in, const std::vector<int> &cols) {
    XH_REQUIRE(!cols.empty() && cols.size() <= MAX_ARITY, XLOG_HIP_INVALID_ARG, "projection needs 1..8 columns");
    xlog_hip_rel *r = rel_new(ctx, (uint32_t)cols.size(), in->rows);
    r->rows = in->rows;
    ProjSpec s{(int)in->arity, (int)cols.size(), {0, 0, 0, 0, 0, 0, 0, 0}};
    for (size_t i = 0; i < cols.size(); ++i) s.cols[i] = cols[i];
    LAUNCH_1D(k_project, in->rows, view_of(in), in->rows, s, out_of(r));
    return r;
}

// a positive integer from the environment, or dflt
uint64_t env_u64(const char *name, uint64_t dflt) {
    const char *e = getenv(name);
    if (e && *e) {
        const unsigned long long v = strtoull(e, nullptr, 10);
        if (v > 0) return v;
    }
    return dflt;
}

}  // namespace xh

// ===========================================================================
// C ABI
// ===========================================================================
using namespace xh;

struct xlog_hip_ctx {
    Ctx c;
};

static Ctx *C(xlog_hip_ctx *ctx) {
    XH_REQUIRE(ctx, XLOG_HIP_INVALID_ARG, "context is NULL");
    XH_CHECK_HIP(hipSetDevice(ctx->c.device));
    return &ctx->c;
}
static void need_rel(const xlog_hip_rel *r, const char *what) {
    XH_REQUIRE(r, XLOG_HIP_INVALID_ARG, std::string(what) + " is NULL");
}

namespace xh {
// Arrow IPC stream I/O helpers (provider/io.rs:697-773)
namespace {
// Device relation from UInt32 column buffers in host memory: each column is
// copied once to a device staging buffer and packed there.
xlog_hip_rel *rel_from_ipc(Ctx *ctx, const IpcColumns &ic) {
    xlog_hip_rel *r = rel_new(ctx, ic.arity, ic.rows);
    r->rows = ic.rows;
    if (!ic.rows) return r;
    try {
        Buf<uint32_t> stage(ctx, (uint64_t)ic.arity * ic.rows);
        const uint32_t *dc[MAX_ARITY] = {nullptr};
        for (uint32_t c = 0; c < ic.arity; ++c) {
            uint32_t *d = stage.p + (uint64_t)c * ic.rows;
            XH_CHECK_HIP(hipMemcpyAsync(d, ic.cols[c], ic.rows * 4, hipMemcpyHostToDevice, ctx->stream));
            dc[c] = d;
        }
        pack_device_columns(ctx, dc, ic.arity, ic.rows, r);
        ctx->sync();  // the host bytes may go away after the call
    } catch (...) {
        rel_free(r);
        throw;
    }
    return r;
}

// All columns of a relation, column-major in host memory
std::vector<uint32_t> columns_to_host(Ctx *ctx, const xlog_hip_rel *rel) {
    std::vector<uint32_t> h((uint64_t)rel->arity * rel->rows);
    if (!rel->rows) return h;
    Buf<uint32_t> tmp(ctx, (uint64_t)rel->arity * rel->rows);
    for (uint32_t c = 0; c < rel->arity; ++c) {
        uint32_t *d = tmp.p + (uint64_t)c * rel->rows;
        if (rel->arity == 1) LAUNCH_1D(k_u64_to_u32, rel->rows, rel->w[0], rel->rows, d);
        else unpack_column(ctx, rel->w[c / 2], (c % 2) == 0, rel->rows, d);
    }
    XH_CHECK_HIP(hipMemcpyAsync(h.data(), tmp.p, h.size() * 4, hipMemcpyDeviceToHost, ctx->stream));
    ctx->sync();
    return h;
}

std::vector<uint8_t> rel_to_ipc(Ctx *ctx, const xlog_hip_rel *rel, const char *const *names) {
    const std::vector<uint32_t> h = columns_to_host(ctx, rel);
    const uint32_t *cols[4] = {nullptr, nullptr, nullptr, nullptr};
    for (uint32_t c = 0; c < rel->arity; ++c) cols[c] = h.data() + (uint64_t)c * rel->rows;
    return ipc_encode_u32(cols, rel->arity, rel->rows, names);
}

uint8_t *to_malloc(const std::vector<uint8_t> &v) {
    uint8_t *p = static_cast<uint8_t *>(malloc(v.size() ? v.size() : 1));
    XH_REQUIRE(p, XLOG_HIP_OOM, "host allocation failed");
    if (!v.empty()) memcpy(p, v.data(), v.size());
    return p;
}
}  // namespace
}  // namespace xh

extern "C" {

const char *xlog_hip_last_error(void) { return g_last_error.c_str(); }
const char *xlog_hip_version(void) { return "xlog_hip 0.1.0 (gfx950)"; }

xlog_hip_status xlog_hip_ctx_create(int device, xlog_hip_ctx **out) {
    return guarded([&] {
        XH_REQUIRE(out, XLOG_HIP_INVALID_ARG, "out is NULL");
        *out = nullptr;
        int count = 0;
        XH_CHECK_HIP(hipGetDeviceCount(&count));
        XH_REQUIRE(device >= 0 && device < count, XLOG_HIP_INVALID_ARG, "device index out of range");
        XH_CHECK_HIP(hipSetDevice(device));
        std::unique_ptr<xlog_hip_ctx> h(new xlog_hip_ctx());
        Ctx &c = h->c;
        c.device = device;
        hipDeviceProp_t prop;
        XH_CHECK_HIP(hipGetDeviceProperties(&prop, device));
        c.num_cus = prop.multiProcessorCount;
        XH_CHECK_HIP(hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking));
        c.pool = new Pool(device);
        XH_CHECK_HIP(hipHostMalloc((void **)&c.host_scalars, Ctx::HOST_STAGE_U64 * sizeof(uint64_t),
                                   hipHostMallocDefault));
        scan_noalloc_init(device);  // the allocation-free scan's scratch on this device
        c.tickets = static_cast<unsigned long long *>(c.alloc(16 * sizeof(unsigned long long)));
        fill_u64(&c, reinterpret_cast<uint64_t *>(c.tickets), 0ull, 16);
        XH_CHECK_HIP(hipEventCreate(&c.ev_a));
        XH_CHECK_HIP(hipEventCreate(&c.ev_b));
        XH_CHECK_HIP(hipEventCreateWithFlags(&c.ev_sync, hipEventDisableTiming));
        XH_CHECK_HIP(hipEventCreateWithFlags(&c.ev_read, hipEventDisableTiming));
        c.sync();
        *out = h.release();
    });
}

void xlog_hip_ctx_destroy(xlog_hip_ctx *ctx) {
    if (!ctx) return;
    Ctx &c = ctx->c;
    (void)hipSetDevice(c.device);
    (void)hipStreamSynchronize(c.stream);
    sort_state_release(&c);
    select_state_release(&c);
    if (c.tickets) c.free(c.tickets);
    if (c.prof_work) c.free(c.prof_work);
    delete c.pool;
    if (c.host_scalars) (void)hipHostFree(c.host_scalars);
    if (c.ev_a) (void)hipEventDestroy(c.ev_a);
    if (c.ev_b) (void)hipEventDestroy(c.ev_b);
    if (c.ev_sync) (void)hipEventDestroy(c.ev_sync);
    if (c.ev_read) (void)hipEventDestroy(c.ev_read);
    for (auto &r : c.prof_pending) {
        (void)hipEventDestroy(r.a);
        (void)hipEventDestroy(r.b);
    }
    for (hipEvent_t e : c.prof_events) (void)hipEventDestroy(e);
    (void)hipStreamDestroy(c.stream);
    delete ctx;
}

xlog_hip_status xlog_hip_synchronize(xlog_hip_ctx *ctx) { return guarded([&] { C(ctx)->sync(); }); }
void *xlog_hip_stream(xlog_hip_ctx *ctx) { return ctx ? (void *)ctx->c.stream : nullptr; }

xlog_hip_status xlog_hip_memory_stats(xlog_hip_ctx *ctx, uint64_t *in_use, uint64_t *peak, uint64_t *cached) {
    return guarded([&] {
        Ctx *c = C(ctx);
        if (in_use) *in_use = c->pool->bytes_in_use();
        if (peak) *peak = c->pool->peak_in_use();
        if (cached) *cached = c->pool->bytes_cached();
    });
}
xlog_hip_status xlog_hip_trim(xlog_hip_ctx *ctx) { return guarded([&] { C(ctx)->pool->trim(); }); }
xlog_hip_status xlog_hip_set_memory_budget(xlog_hip_ctx *ctx, uint64_t device_bytes) {
    return guarded([&] {
        Ctx *c = C(ctx);
        c->pool->set_budget((size_t)device_bytes);
        if (device_bytes && c->pool->bytes_in_use() + c->pool->bytes_cached() > device_bytes) c->pool->trim();
    });
}

xlog_hip_status xlog_hip_rel_create_empty(xlog_hip_ctx *ctx, uint32_t arity, xlog_hip_rel **out) {
    return guarded([&] {
        XH_REQUIRE(out, XLOG_HIP_INVALID_ARG, "out is NULL");
        *out = rel_new(C(ctx), arity, 0);
        (*out)->flags = REL_CANONICAL;
    });
}

xlog_hip_status xlog_hip_rel_from_host_columns(xlog_hip_ctx *ctx, const uint32_t *const *cols, uint32_t arity,
                                               uint64_t rows, xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        XH_REQUIRE(out, XLOG_HIP_INVALID_ARG, "out is NULL");
        XH_REQUIRE(arity >= 1 && arity <= MAX_ARITY, XLOG_HIP_INVALID_ARG, "relation arity must be 1..8");
        XH_REQUIRE(rows == 0 || cols, XLOG_HIP_INVALID_ARG, "columns are NULL");
        for (uint32_t i = 0; i < arity && rows; ++i) XH_REQUIRE(cols[i], XLOG_HIP_INVALID_ARG, "column pointer is NULL");
        const int nw = words_for(arity);
        std::vector<std::vector<uint64_t>> h(nw, std::vector<uint64_t>(rows));
        for (uint64_t i = 0; i < rows; ++i) {
            if (arity == 1) {
                h[0][i] = cols[0][i];
                continue;
            }
            for (int k = 0; k < nw; ++k)
                h[k][i] = ((uint64_t)cols[2 * k][i] << 32) | (2u * k + 1 < arity ? cols[2 * k + 1][i] : 0u);
        }
        std::unique_ptr<xlog_hip_rel, void (*)(xlog_hip_rel *)> r(rel_new(c, arity, rows), rel_free);
        r->rows = rows;
        if (rows)
            for (int k = 0; k < nw; ++k)
                XH_CHECK_HIP(hipMemcpyAsync(r->w[k], h[k].data(), rows * 8, hipMemcpyHostToDevice, c->stream));
        c->sync();
        *out = r.release();
    });
}

xlog_hip_status xlog_hip_rel_from_device_columns(xlog_hip_ctx *ctx, const uint32_t *const *dev_cols, uint32_t arity,
                                                 uint64_t rows, xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *ctxp = C(ctx);
        Ctx *ctx = ctxp;
        XH_REQUIRE(out, XLOG_HIP_INVALID_ARG, "out is NULL");
        XH_REQUIRE(arity >= 1 && arity <= MAX_ARITY, XLOG_HIP_INVALID_ARG, "relation arity must be 1..8");
        XH_REQUIRE(rows == 0 || dev_cols, XLOG_HIP_INVALID_ARG, "columns are NULL");
        xlog_hip_rel *r = rel_new(ctx, arity, rows);
        r->rows = rows;
        if (rows) pack_device_columns(ctx, dev_cols, arity, rows, r);
        *out = r;
    });
}

xlog_hip_status xlog_hip_rel_from_host_packed(xlog_hip_ctx *ctx, const uint64_t *keys, uint32_t arity, uint64_t rows,
                                              xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        XH_REQUIRE(out, XLOG_HIP_INVALID_ARG, "out is NULL");
        XH_REQUIRE(arity == 1 || arity == 2, XLOG_HIP_INVALID_ARG, "packed upload supports arity 1 or 2");
        XH_REQUIRE(rows == 0 || keys, XLOG_HIP_INVALID_ARG, "keys are NULL");
        xlog_hip_rel *r = rel_new(c, arity, rows);
        r->rows = rows;
        if (rows) XH_CHECK_HIP(hipMemcpyAsync(r->w[0], keys, rows * 8, hipMemcpyHostToDevice, c->stream));
        c->sync();
        *out = r;
    });
}

xlog_hip_status xlog_hip_rel_download_column(xlog_hip_ctx *ctx, const xlog_hip_rel *rel, uint32_t col, uint32_t *host,
                                             uint64_t host_cap) {
    return guarded([&] {
        Ctx *ctxp = C(ctx);
        Ctx *ctx = ctxp;
        need_rel(rel, "relation");
        XH_REQUIRE(col < rel->arity, XLOG_HIP_INVALID_ARG, "column out of range");
        XH_REQUIRE(host_cap >= rel->rows, XLOG_HIP_CAPACITY_OVERFLOW, "host buffer too small");
        if (!rel->rows) return;
        XH_REQUIRE(host, XLOG_HIP_INVALID_ARG, "host buffer is NULL");
        Buf<uint32_t> tmp(ctx, rel->rows);
        if (rel->arity == 1) LAUNCH_1D(k_u64_to_u32, rel->rows, rel->w[0], rel->rows, tmp.p);
        else {
            unpack_column(ctx, rel->w[col / 2], (col % 2) == 0, rel->rows, tmp.p);
        }
        XH_CHECK_HIP(hipMemcpyAsync(host, tmp.p, rel->rows * 4, hipMemcpyDeviceToHost, ctx->stream));
        ctx->sync();
    });
}


// ---- Arrow IPC stream I/O (provider/io.rs:697-773) ----------------------------
xlog_hip_status xlog_hip_arrow_ipc_decode_u32(const uint8_t *ipc, uint64_t len, uint32_t *arity, uint64_t *rows,
                                              uint32_t *cols, uint64_t cols_cap) {
    return guarded([&] {
        XH_REQUIRE(arity && rows, XLOG_HIP_INVALID_ARG, "arity / rows is NULL");
        IpcColumns ic;
        ipc_decode_u32(ipc, len, ic);
        *arity = ic.arity;
        *rows = ic.rows;
        if (!cols) return;
        XH_REQUIRE(cols_cap >= (uint64_t)ic.arity * ic.rows, XLOG_HIP_CAPACITY_OVERFLOW, "column buffer too small");
        for (uint32_t c = 0; c < ic.arity; ++c) memcpy(cols + (uint64_t)c * ic.rows, ic.cols[c], ic.rows * 4);
    });
}

xlog_hip_status xlog_hip_arrow_ipc_encode_u32(const uint32_t *const *cols, uint32_t arity, uint64_t rows,
                                              const char *const *names, uint8_t **ipc, uint64_t *len) {
    return guarded([&] {
        XH_REQUIRE(ipc && len, XLOG_HIP_INVALID_ARG, "ipc / len is NULL");
        const std::vector<uint8_t> v = ipc_encode_u32(cols, arity, rows, names);
        *ipc = to_malloc(v);
        *len = v.size();
    });
}

void xlog_hip_bytes_free(uint8_t *p) { free(p); }

xlog_hip_status xlog_hip_rel_from_arrow_ipc(xlog_hip_ctx *ctx, const uint8_t *ipc, uint64_t len, xlog_hip_rel **out) {
    return guarded([&] {
        XH_REQUIRE(out, XLOG_HIP_INVALID_ARG, "out is NULL");
        IpcColumns ic;
        ipc_decode_u32(ipc, len, ic);
        *out = rel_from_ipc(C(ctx), ic);
    });
}

xlog_hip_status xlog_hip_rel_to_arrow_ipc(xlog_hip_ctx *ctx, const xlog_hip_rel *rel, const char *const *names,
                                          uint8_t **ipc, uint64_t *len) {
    return guarded([&] {
        need_rel(rel, "relation");
        XH_REQUIRE(ipc && len, XLOG_HIP_INVALID_ARG, "ipc / len is NULL");
        const std::vector<uint8_t> v = rel_to_ipc(C(ctx), rel, names);
        *ipc = to_malloc(v);
        *len = v.size();
    });
}

xlog_hip_status xlog_hip_read_arrow_ipc_stream_file(xlog_hip_ctx *ctx, const char *path, xlog_hip_rel **out) {
    return guarded([&] {
        XH_REQUIRE(path && out, XLOG_HIP_INVALID_ARG, "path / out is NULL");
        const std::string where = std::string("Failed to read Arrow IPC stream from ") + path + ": ";
        const int fd = open(path, O_RDONLY);
        XH_REQUIRE(fd >= 0, XLOG_HIP_INVALID_ARG, where + strerror(errno));
        struct stat st;
        if (fstat(fd, &st) != 0) {
            const int e = errno;
            close(fd);
            throw Error{XLOG_HIP_INVALID_ARG, where + strerror(e)};
        }
        const uint64_t n = (uint64_t)st.st_size;
        void *m = n ? mmap(nullptr, n, PROT_READ, MAP_PRIVATE, fd, 0) : nullptr;
        close(fd);
        XH_REQUIRE(n == 0 || m != MAP_FAILED, XLOG_HIP_INVALID_ARG, where + strerror(errno));
        // the column buffers are uploaded straight from the mapping
        try {
            IpcColumns ic;
            ipc_decode_u32(static_cast<const uint8_t *>(m), n, ic);
            *out = rel_from_ipc(C(ctx), ic);
        } catch (...) {
            if (m) munmap(m, n);
            throw;
        }
        if (m) munmap(m, n);
    });
}

xlog_hip_status xlog_hip_write_arrow_ipc_stream_file(xlog_hip_ctx *ctx, const xlog_hip_rel *rel,
                                                     const char *const *names, const char *path) {
    return guarded([&] {
        need_rel(rel, "relation");
        XH_REQUIRE(path, XLOG_HIP_INVALID_ARG, "path is NULL");
        const std::vector<uint8_t> v = rel_to_ipc(C(ctx), rel, names);
        const std::string where = std::string("Failed to write Arrow IPC stream to ") + path + ": ";
        FILE *f = fopen(path, "wb");
        XH_REQUIRE(f, XLOG_HIP_INVALID_ARG, where + strerror(errno));
        const bool wrote = v.empty() || fwrite(v.data(), 1, v.size(), f) == v.size();
        const int e = errno;
        const bool closed = fclose(f) == 0;
        XH_REQUIRE(wrote && closed, XLOG_HIP_INVALID_ARG, where + strerror(wrote ? errno : e));
    });
}

xlog_hip_status xlog_hip_rel_download_packed(xlog_hip_ctx *ctx, const xlog_hip_rel *rel, uint64_t *host,
                                             uint64_t host_cap) {
    return guarded([&] {
        Ctx *c = C(ctx);
        need_rel(rel, "relation");
        XH_REQUIRE(rel->arity <= 2, XLOG_HIP_INVALID_ARG, "packed download supports arity 1 or 2");
        XH_REQUIRE(host_cap >= rel->rows, XLOG_HIP_CAPACITY_OVERFLOW, "host buffer too small");
        if (!rel->rows) return;
        XH_REQUIRE(host, XLOG_HIP_INVALID_ARG, "host buffer is NULL");
        XH_CHECK_HIP(hipMemcpyAsync(host, rel->w[0], rel->rows * 8, hipMemcpyDeviceToHost, c->stream));
        c->sync();
    });
}

xlog_hip_status xlog_hip_rel_num_rows(const xlog_hip_rel *rel, uint64_t *rows) {
    return guarded([&] {
        need_rel(rel, "relation");
        XH_REQUIRE(rows, XLOG_HIP_INVALID_ARG, "rows is NULL");
        *rows = rel->rows;
    });
}
xlog_hip_status xlog_hip_rel_arity(const xlog_hip_rel *rel, uint32_t *arity) {
    return guarded([&] {
        need_rel(rel, "relation");
        XH_REQUIRE(arity, XLOG_HIP_INVALID_ARG, "arity is NULL");
        *arity = rel->arity;
    });
}
xlog_hip_status xlog_hip_rel_is_canonical(const xlog_hip_rel *rel, int *canonical) {
    return guarded([&] {
        need_rel(rel, "relation");
        XH_REQUIRE(canonical, XLOG_HIP_INVALID_ARG, "canonical is NULL");
        *canonical = (rel->flags & REL_CANONICAL) ? 1 : 0;
    });
}
xlog_hip_status xlog_hip_rel_device_words(const xlog_hip_rel *rel, uint32_t word, const uint64_t **dev) {
    return guarded([&] {
        need_rel(rel, "relation");
        XH_REQUIRE(dev, XLOG_HIP_INVALID_ARG, "dev is NULL");
        XH_REQUIRE(word < (uint32_t)rel->nwords(), XLOG_HIP_INVALID_ARG, "word index out of range");
        *dev = rel->w[word];
    });
}
xlog_hip_status xlog_hip_rel_clone(xlog_hip_ctx *ctx, const xlog_hip_rel *in, xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        need_rel(in, "input");
        XH_REQUIRE(out, XLOG_HIP_INVALID_ARG, "out is NULL");
        *out = rel_clone(c, in);
    });
}
void xlog_hip_rel_free(xlog_hip_rel *rel) {
    if (rel && rel->ctx) (void)hipSetDevice(rel->ctx->device);
    rel_free(rel);
}

#define OUT_GUARD XH_REQUIRE(out, XLOG_HIP_INVALID_ARG, "out is NULL"); *out = nullptr

xlog_hip_status xlog_hip_sort(xlog_hip_ctx *ctx, const xlog_hip_rel *in, const uint32_t *key_cols, uint32_t n_keys,
                              xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        need_rel(in, "input");
        *out = op_sort(c, in, check_cols(in, key_cols, n_keys));
    });
}
xlog_hip_status xlog_hip_dedup(xlog_hip_ctx *ctx, const xlog_hip_rel *in, const uint32_t *key_cols, uint32_t n_keys,
                               xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        need_rel(in, "input");
        *out = op_dedup(c, in, check_cols(in, key_cols, n_keys));
    });
}
xlog_hip_status xlog_hip_dedup_full_row(xlog_hip_ctx *ctx, const xlog_hip_rel *in, xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        need_rel(in, "input");
        *out = op_dedup_full(c, in);
    });
}
xlog_hip_status xlog_hip_union(xlog_hip_ctx *ctx, const xlog_hip_rel *a, const xlog_hip_rel *b, xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        need_rel(a, "a");
        need_rel(b, "b");
        const xlog_hip_rel *ins[2] = {a, b};
        *out = op_union_many(c, ins, 2);
    });
}
xlog_hip_status xlog_hip_union_many(xlog_hip_ctx *ctx, const xlog_hip_rel *const *ins, uint32_t n_ins,
                                    xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        *out = op_union_many(c, ins, n_ins);
    });
}
xlog_hip_status xlog_hip_diff(xlog_hip_ctx *ctx, const xlog_hip_rel *a, const xlog_hip_rel *b, xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        need_rel(a, "a");
        need_rel(b, "b");
        *out = op_diff(c, a, b);
    });
}
xlog_hip_status xlog_hip_hash_join(xlog_hip_ctx *ctx, const xlog_hip_rel *left, const xlog_hip_rel *right,
                                   uint32_t left_key, uint32_t right_key, int join_type, xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        *out = op_join(c, left, right, left_key, right_key, join_type, nullptr);
    });
}
xlog_hip_status xlog_hip_hash_join_keys(xlog_hip_ctx *ctx, const xlog_hip_rel *left, const xlog_hip_rel *right,
                                        const uint32_t *left_keys, const uint32_t *right_keys, uint32_t n_keys,
                                        int join_type, xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        need_rel(left, "left");
        need_rel(right, "right");
        XH_REQUIRE(n_keys >= 1 && left_keys && right_keys, XLOG_HIP_INVALID_ARG, "key column lists are empty or NULL");
        XH_REQUIRE(n_keys <= MAX_ARITY, XLOG_HIP_INVALID_ARG, "more key columns than columns");
        std::vector<int> lk(left_keys, left_keys + n_keys), rk(right_keys, right_keys + n_keys);
        for (uint32_t t = 0; t < n_keys; ++t)
            XH_REQUIRE(left_keys[t] < left->arity && right_keys[t] < right->arity, XLOG_HIP_INVALID_ARG,
                       "join key column out of range");
        if (n_keys == 1 && left->arity <= 2 && right->arity <= 2)
            *out = op_join(c, left, right, left_keys[0], right_keys[0], join_type, nullptr);
        else
            *out = op_join_keys(c, left, right, lk, rk, join_type);
    });
}
xlog_hip_status xlog_hip_join_index_build(xlog_hip_ctx *ctx, const xlog_hip_rel *right, const uint32_t *right_keys,
                                          uint32_t n_keys, xlog_hip_join_index **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        need_rel(right, "right");
        XH_REQUIRE(n_keys >= 1 && right_keys, XLOG_HIP_INVALID_ARG, "Join requires at least one key column");
        XH_REQUIRE(n_keys <= MAX_ARITY, XLOG_HIP_INVALID_ARG, "more key columns than columns");
        for (uint32_t t = 0; t < n_keys; ++t)
            XH_REQUIRE(right_keys[t] < right->arity, XLOG_HIP_INVALID_ARG, "right key column out of range");
        XH_REQUIRE(right->rows > 0, XLOG_HIP_INVALID_ARG, "cannot build a join index for an empty relation");
        XH_REQUIRE(right->rows < KEY_NONE, XLOG_HIP_CAPACITY_OVERFLOW, "join: more than 2^32 - 2 rows on one side");
        std::unique_ptr<xlog_hip_join_index> ix(new xlog_hip_join_index);
        ix->ctx = c;
        ix->arity = right->arity;
        ix->keys.assign(right_keys, right_keys + n_keys);
        ix->rows = right->rows;
        if (n_keys == 1 && right->arity <= 2) {
            build_join_index(c, right->w[0], right->rows, right->arity, (int)right_keys[0],
                             (right->flags & REL_CANONICAL) != 0, ix->J);
        } else {
            ix->F.reset(new KeyFold());
            fold_build(c, right, std::vector<int>(right_keys, right_keys + n_keys), *ix->F, true);
        }
        *out = ix.release();
    });
}
xlog_hip_status xlog_hip_hash_join_with_index(xlog_hip_ctx *ctx, const xlog_hip_rel *left, const xlog_hip_rel *right,
                                              const uint32_t *left_keys, const uint32_t *right_keys, uint32_t n_keys,
                                              int join_type, const xlog_hip_join_index *index, uint64_t max_output,
                                              xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        need_rel(left, "left");
        need_rel(right, "right");
        XH_REQUIRE(index, XLOG_HIP_INVALID_ARG, "join index is NULL");
        XH_REQUIRE(index->ctx == c, XLOG_HIP_INVALID_ARG, "join index belongs to another context");
        XH_REQUIRE(n_keys >= 1 && left_keys && right_keys, XLOG_HIP_INVALID_ARG,
                   "Join requires at least one key column");
        XH_REQUIRE(n_keys <= MAX_ARITY, XLOG_HIP_INVALID_ARG, "more key columns than columns");
        std::vector<int> lk(left_keys, left_keys + n_keys), rk(right_keys, right_keys + n_keys);
        check_key_lists(left, right, lk, rk, join_type);
        // the index must have been built over this right relation and these key columns (relational.rs:3975-3985)
        XH_REQUIRE(index->rows == right->rows, XLOG_HIP_INVALID_ARG,
                   "Join index row count does not match right relation");
        XH_REQUIRE(index->arity == right->arity &&
                       std::vector<uint32_t>(right_keys, right_keys + n_keys) == index->keys,
                   XLOG_HIP_INVALID_ARG, "Join index key columns do not match requested right_keys");
        if (left->rows == 0) {
            *out = empty_side_join(c, left, right, join_type);
            return;
        }
        if (index->F) {
            *out = keyed_join_probe(c, left, right, lk, *index->F, join_type, max_output);
        } else if (left->arity <= 2) {
            *out = op_join_indexed(c, left, left_keys[0], index->J, right->arity, right_keys[0], join_type, nullptr,
                                   max_output);
        } else {
            *out = direct_join_wide_left(c, left, left_keys[0], index->J, right->arity, right_keys[0], join_type,
                                         max_output);
        }
    });
}
void xlog_hip_join_index_free(xlog_hip_join_index *index) { delete index; }
xlog_hip_status xlog_hip_nested_loop_join(xlog_hip_ctx *ctx, const xlog_hip_rel *left, const xlog_hip_rel *right,
                                          uint32_t left_key, uint32_t right_key, xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        *out = op_nested_loop_join(c, left, right, left_key, right_key);
    });
}
xlog_hip_status xlog_hip_dedup_sorted(xlog_hip_ctx *ctx, const xlog_hip_rel *in, const uint32_t *key_cols,
                                      uint32_t n_keys, xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        need_rel(in, "input");
        *out = op_dedup_sorted(c, in, check_cols(in, key_cols, n_keys));
    });
}
xlog_hip_status xlog_hip_fj_delta_novel(xlog_hip_ctx *ctx, const xlog_hip_rel *delta, const xlog_hip_rel *edge,
                                        const xlog_hip_rel *full, const xlog_hip_fj_delta_cols *cols, uint32_t domain,
                                        xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        XH_REQUIRE(cols, XLOG_HIP_INVALID_ARG, "column roles are NULL");
        *out = op_fj_delta(c, delta, edge, full, *cols, domain);
    });
}
xlog_hip_status xlog_hip_fj_delta_sparse_novel(xlog_hip_ctx *ctx, const xlog_hip_rel *delta, const xlog_hip_rel *edge,
                                               const xlog_hip_rel *full, const xlog_hip_fj_delta_cols *cols,
                                               uint64_t max_table_bytes, xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        XH_REQUIRE(cols, XLOG_HIP_INVALID_ARG, "cols is NULL");
        need_rel(delta, "delta");
        need_rel(edge, "edge");
        need_rel(full, "full");
        bool declined = false;
        xlog_hip_rel *r = op_fj_delta_sparse(c, delta, edge, full, *cols, max_table_bytes, &declined);
        *out = declined ? nullptr : r;
    });
}
xlog_hip_status xlog_hip_sort_merge_join(xlog_hip_ctx *ctx, const xlog_hip_rel *left, const xlog_hip_rel *right,
                                         uint32_t left_key, uint32_t right_key, xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        *out = op_sort_merge_join(c, left, right, left_key, right_key);
    });
}
xlog_hip_status xlog_hip_join_project(xlog_hip_ctx *ctx, const xlog_hip_rel *left, const xlog_hip_rel *right,
                                      uint32_t left_key, uint32_t right_key, const uint32_t *out_cols, uint32_t n_out,
                                      xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        XH_REQUIRE(out_cols && n_out >= 1 && n_out <= 4, XLOG_HIP_INVALID_ARG, "out_cols must list 1..4 columns");
        std::vector<int> oc(out_cols, out_cols + n_out);
        *out = op_join(c, left, right, left_key, right_key, XLOG_HIP_JOIN_INNER, &oc);
    });
}
xlog_hip_status xlog_hip_join_project_dedup(xlog_hip_ctx *ctx, const xlog_hip_rel *left, const xlog_hip_rel *right,
                                            uint32_t left_key, uint32_t right_key, const uint32_t *out_cols,
                                            uint32_t n_out, xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        XH_REQUIRE(out_cols && n_out >= 1 && n_out <= 4, XLOG_HIP_INVALID_ARG, "out_cols must list 1..4 columns");
        std::vector<int> oc(out_cols, out_cols + n_out);
        *out = op_join_project_dedup(c, left, right, left_key, right_key, oc);
    });
}
xlog_hip_status xlog_hip_project(xlog_hip_ctx *ctx, const xlog_hip_rel *in, const uint32_t *cols, uint32_t n_cols,
                                 xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        need_rel(in, "input");
        *out = op_project(c, in, check_cols(in, cols, n_cols));
    });
}
xlog_hip_status xlog_hip_is_sorted(xlog_hip_ctx *ctx, const xlog_hip_rel *rel, uint32_t col, int *sorted) {
    return guarded([&] {
        Ctx *c = C(ctx);
        need_rel(rel, "relation");
        XH_REQUIRE(sorted, XLOG_HIP_INVALID_ARG, "sorted is NULL");
        XH_REQUIRE(col < rel->arity, XLOG_HIP_INVALID_ARG, "column out of range");
        *sorted = column_sorted(c, rel, col) ? 1 : 0;
    });
}
xlog_hip_status xlog_hip_exclusive_scan_u32(xlog_hip_ctx *ctx, uint32_t *dev, uint64_t n, uint64_t *total) {
    return guarded([&] {
        Ctx *ctxp = C(ctx);
        Ctx *ctx = ctxp;
        XH_REQUIRE(n == 0 || dev, XLOG_HIP_INVALID_ARG, "array is NULL");
        if (n == 0) { if (total) *total = 0; return; }
        Buf<unsigned long long> tot(ctx, 1);
        scan_u32_inplace(ctx, dev, n, tot.p);
        ctx->read_scalars(tot.p, 1);
        if (total) *total = ctx->host_scalars[0];
    });
}
xlog_hip_status xlog_hip_exclusive_scan_u32_noalloc(xlog_hip_ctx *ctx, uint32_t *dev, uint64_t n, uint64_t *total) {
    return guarded([&] {
        Ctx *c = C(ctx);
        XH_REQUIRE(n == 0 || dev, XLOG_HIP_INVALID_ARG, "array is NULL");
        scan_u32_inplace_noalloc(c, dev, n, total);
    });
}
xlog_hip_status xlog_hip_compact(xlog_hip_ctx *ctx, const xlog_hip_rel *in, const uint8_t *dev_mask, xlog_hip_rel **out) {
    return guarded([&] {
        Ctx *c = C(ctx);
        OUT_GUARD;
        need_rel(in, "input");
        XH_REQUIRE(in->rows == 0 || dev_mask, XLOG_HIP_INVALID_ARG, "mask is NULL");
        *out = compact_rel(c, in, dev_mask);
        if (in->flags & REL_CANONICAL) (*out)->flags = REL_CANONICAL;
    });
}

xlog_hip_status xlog_hip_fixpoint(xlog_hip_ctx *ctx, const int32_t *plan, uint32_t n_preds,
                                  const xlog_hip_rel *const *rels, xlog_hip_rel **out, xlog_hip_fixpoint_stats *stats) {
    return guarded([&] { run_fixpoint(C(ctx), plan, n_preds, rels, out, stats); });
}

xlog_hip_status xlog_hip_fixpoint_tc(xlog_hip_ctx *ctx, const xlog_hip_rel *edge, xlog_hip_rel **reach,
                                     xlog_hip_fixpoint_stats *stats) {
    return guarded([&] {
        Ctx *c = C(ctx);
        need_rel(edge, "edge");
        XH_REQUIRE(reach, XLOG_HIP_INVALID_ARG, "reach is NULL");
        // preds: 0 = edge, 1 = reach ; vars X=0 Y=1 Z=2
        static const int32_t plan[] = {2, 1, 0, 1, 1, 0, 0, 1, 1, 0, 2, 2, 1, 0, 1, 0, 1, 2};
        const xlog_hip_rel *rels[2] = {edge, nullptr};
        xlog_hip_rel *outs[2] = {nullptr, nullptr};
        run_fixpoint(c, plan, 2, rels, outs, stats);
        *reach = outs[1];
    });
}

xlog_hip_status xlog_hip_rel_digest(xlog_hip_ctx *ctx, const xlog_hip_rel *rel, uint64_t *digest) {
    return guarded([&] {
        Ctx *c = C(ctx);
        need_rel(rel, "relation");
        XH_REQUIRE(digest, XLOG_HIP_INVALID_ARG, "digest is NULL");
        XH_REQUIRE(rel->arity <= 2, XLOG_HIP_UNSUPPORTED, "digest supports arity 1 or 2");
        std::vector<uint64_t> h(rel->rows);
        if (rel->rows) {
            XH_CHECK_HIP(hipMemcpyAsync(h.data(), rel->w[0], rel->rows * 8, hipMemcpyDeviceToHost, c->stream));
            c->sync();
        }
        uint64_t x = 0xcbf29ce484222325ULL;
        for (uint64_t k : h)
            for (int b = 0; b < 8; ++b) { x ^= (k >> (8 * b)) & 255; x *= 0x100000001b3ULL; }
        *digest = x;
    });
}

}  // extern "C"

// ---- kernel timing -----------------------------------------------------------
unsigned long long *xh::Prof::work(double bytes_per_unit) {
    if (!on) return nullptr;
    constexpr uint64_t total = (uint64_t)Ctx::PROF_WORK_SLOTS * Ctx::PROF_WORK_SPREAD;
    if (!ctx->prof_work) {
        ctx->prof_work = static_cast<unsigned long long *>(ctx->alloc(total * sizeof(uint64_t)));
        fill_u64(ctx, reinterpret_cast<uint64_t *>(ctx->prof_work), 0ull, total);
    }
    if (ctx->prof_work_next >= Ctx::PROF_WORK_SLOTS) return nullptr;
    rec.work_slot = ctx->prof_work_next++;
    rec.bytes_per_work = bytes_per_unit;
    return ctx->prof_work + (uint64_t)rec.work_slot * Ctx::PROF_WORK_SPREAD;
}

void xh::Ctx::prof_resolve() {
    if (prof_pending.empty()) return;
    sync();
    std::vector<uint64_t> work;
    if (prof_work_next > 0) {
        const uint64_t n = (uint64_t)prof_work_next * PROF_WORK_SPREAD;
        std::vector<uint64_t> raw(n);
        XH_CHECK_HIP(hipMemcpy(raw.data(), prof_work, n * sizeof(uint64_t), hipMemcpyDeviceToHost));
        fill_u64(this, reinterpret_cast<uint64_t *>(prof_work), 0ull, n);
        work.assign(prof_work_next, 0);
        for (uint64_t i = 0; i < n; ++i) work[i / PROF_WORK_SPREAD] += raw[i];
        prof_work_next = 0;
    }
    for (auto &r : prof_pending) {
        float ms = 0.f;
        XH_CHECK_HIP(hipEventElapsedTime(&ms, r.a, r.b));
        if (r.kind >= 0 && r.kind < XLOG_HIP_KERNEL_KINDS) {
            prof_ms[r.kind] += ms;
            prof_bytes[r.kind] += r.bytes + (r.work_slot >= 0 ? r.bytes_per_work * (double)work[r.work_slot] : 0.0);
            prof_launches[r.kind] += 1;
        }
        prof_events.push_back(r.a);
        prof_events.push_back(r.b);
    }
    prof_pending.clear();
}

extern "C" {
xlog_hip_status xlog_hip_profile_enable(xlog_hip_ctx *ctx, int on) {
    return guarded([&] {
        Ctx *c = C(ctx);
        c->prof_resolve();
        c->profiling = on != 0;
    });
}
xlog_hip_status xlog_hip_profile_reset(xlog_hip_ctx *ctx) {
    return guarded([&] {
        Ctx *c = C(ctx);
        c->prof_resolve();
        for (int k = 0; k < XLOG_HIP_KERNEL_KINDS; ++k) {
            c->prof_ms[k] = 0;
            c->prof_bytes[k] = 0;
            c->prof_launches[k] = 0;
        }
    });
}
xlog_hip_status xlog_hip_profile_read(xlog_hip_ctx *ctx, uint32_t kind, uint64_t *launches, double *total_ms,
                                      double *algo_bytes) {
    return guarded([&] {
        Ctx *c = C(ctx);
        XH_REQUIRE(kind < XLOG_HIP_KERNEL_KINDS, XLOG_HIP_INVALID_ARG, "unknown kernel kind");
        c->prof_resolve();
        if (launches) *launches = c->prof_launches[kind];
        if (total_ms) *total_ms = c->prof_ms[kind];
        if (algo_bytes) *algo_bytes = c->prof_bytes[kind];
    });
}
}  // extern "C"
