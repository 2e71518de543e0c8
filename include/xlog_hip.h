/*
 * xlog_hip.h — C ABI of the MI355X (gfx950) relational core for XLOG's
 * semi-naive Datalog fixpoint.
 *
 * The entry points mirror the inherent methods of the reference's operator
 * provider `xlog_cuda::CudaKernelProvider` (crates/xlog-cuda/src/provider/mod.rs:1139)
 * that the runtime executor (crates/xlog-runtime/src/executor/) calls; each
 * declaration cites the reference method it replaces.
 *
 * Conventions
 *   - Relations are device-resident, u32 columns, arity 1..8.  They are opaque
 *     handles owned by the library; operators borrow inputs (const) and return
 *     new owned relations (reference: every provider op returns a fresh
 *     CudaBuffer, e.g. relational.rs:2219, filter.rs:1927-1933).  Free with
 *     xlog_hip_rel_free().
 *   - Order is lexicographic over columns (col 0 most significant), unsigned per
 *     column; equality is bytewise (kernels/dedup.cu:293-345,398-404).
 *   - Every call returns an xlog_hip_status; on failure the message is
 *     available from xlog_hip_last_error() (thread-local).  No exceptions
 *     cross the ABI.  Errors fail closed like XlogError::Kernel.
 *   - A context owns one HIP stream on one device.  Calls on one context are
 *     stream-ordered; a context must not be used from two threads at once.
 *   - Row counts are uint64_t: the reference's u32 row and 4 GiB column caps
 *     (relational.rs:317-323,773-794,4550-4555) are lifted; results are equal
 *     wherever the reference succeeds.
 */
#ifndef XLOG_HIP_H
#define XLOG_HIP_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    XLOG_HIP_OK = 0,
    XLOG_HIP_INVALID_ARG = 1,
    XLOG_HIP_TYPE_MISMATCH = 2,
    XLOG_HIP_CAPACITY_OVERFLOW = 3,
    XLOG_HIP_ITERATION_LIMIT = 4,
    XLOG_HIP_OOM = 5,
    XLOG_HIP_DEVICE_ERROR = 6,
    XLOG_HIP_UNSUPPORTED = 7
} xlog_hip_status;

typedef struct xlog_hip_ctx xlog_hip_ctx;
typedef struct xlog_hip_rel xlog_hip_rel;
/* reusable join index over a key list of a relation (reference JoinIndexV2) */
typedef struct xlog_hip_join_index xlog_hip_join_index;

/* join kinds (reference JoinType, relational.rs:2926); only INNER is on the path */
#define XLOG_HIP_JOIN_INNER 0
#define XLOG_HIP_JOIN_SEMI 1
#define XLOG_HIP_JOIN_ANTI 2

/* ---- library / context ------------------------------------------------- */

/* Message of the last failed call on this thread ("" if none). */
const char *xlog_hip_last_error(void);
/* Library version string. */
const char *xlog_hip_version(void);

/* Create a context on `device` with its own stream
 * (reference: CudaKernelProvider::new, provider/mod.rs:1139-1242). */
xlog_hip_status xlog_hip_ctx_create(int device, xlog_hip_ctx **out);
/* Destroy a context.  It releases the device memory of every relation and
 * join index still alive on it: those handles must not be passed to any call
 * afterwards, xlog_hip_rel_free / xlog_hip_join_index_free included. */
void xlog_hip_ctx_destroy(xlog_hip_ctx *ctx);
/* Wait for all work of the context (reference: device().synchronize(), executor/mod.rs:1463). */
xlog_hip_status xlog_hip_synchronize(xlog_hip_ctx *ctx);
/* The context's hipStream_t, for callers that order their own work after it. */
void *xlog_hip_stream(xlog_hip_ctx *ctx);
/* Bytes held by live relations and scratch / peak (reference: memory().allocated_bytes(), memory.rs:57-148). */
xlog_hip_status xlog_hip_memory_stats(xlog_hip_ctx *ctx, uint64_t *in_use, uint64_t *peak, uint64_t *cached);
/* Return cached device blocks to the driver. */
xlog_hip_status xlog_hip_trim(xlog_hip_ctx *ctx);
/* Device memory budget of the context in bytes (0: none, the default)
 * (reference: MemoryBudget::with_limit(device_bytes), crates/xlog-core/src/config.rs:39-45,
 * enforced by GpuMemoryManager, crates/xlog-cuda/src/memory.rs:633,756-770, with
 * abort_on_exceed).  An allocation that would take the bytes held by live
 * relations and scratch past it fails with XLOG_HIP_OOM ("GPU memory budget
 * exceeded"), and cached blocks are returned to the driver before the
 * context's footprint would pass it.  The fixpoint's route choice (AUTO) sizes
 * the bitmap routes' matrices against it.  Lowering it below the bytes in use
 * is allowed: later allocations then fail until enough is freed. */
xlog_hip_status xlog_hip_set_memory_budget(xlog_hip_ctx *ctx, uint64_t device_bytes);

/* ---- relations (CudaBuffer counterpart, memory.rs:1758-1930) ------------- */

/* Empty relation of the given arity (reference: create_empty_buffer, provider/mod.rs:3018). */
xlog_hip_status xlog_hip_rel_create_empty(xlog_hip_ctx *ctx, uint32_t arity, xlog_hip_rel **out);
/* Upload host u32 columns (reference: create_buffer_from_slices, provider/io.rs:75). */
xlog_hip_status xlog_hip_rel_from_host_columns(xlog_hip_ctx *ctx, const uint32_t *const *cols, uint32_t arity,
                                               uint64_t rows, xlog_hip_rel **out);
/* Copy device-resident u32 columns into a new relation (no host round trip). */
xlog_hip_status xlog_hip_rel_from_device_columns(xlog_hip_ctx *ctx, const uint32_t *const *dev_cols,
                                                 uint32_t arity, uint64_t rows, xlog_hip_rel **out);
/* Upload host packed keys (arity 2: (c0 << 32) | c1; arity 1: c0). */
xlog_hip_status xlog_hip_rel_from_host_packed(xlog_hip_ctx *ctx, const uint64_t *keys, uint32_t arity,
                                              uint64_t rows, xlog_hip_rel **out);
/* ---- Arrow IPC streams (RecordBatchStream: schema, one record batch, end marker) ----
 * Relations travel as 1..4 UInt32 columns; another column type is TYPE_MISMATCH,
 * compression, dictionaries and big-endian streams are UNSUPPORTED, a stream
 * with no or several record batches is INVALID_ARG (as io.rs:721-737).  Values
 * are taken as stored, validity bitmaps ignored (io.rs:651-653).  Written
 * fields are non-nullable UInt32, named by `names` (NULL: "c0", "c1", ...). */
/* Decode a stream held in host memory into arity x rows column-major u32 values
 * in cols (cols NULL: only *arity and *rows); no device involved. */
xlog_hip_status xlog_hip_arrow_ipc_decode_u32(const uint8_t *ipc, uint64_t len, uint32_t *arity, uint64_t *rows,
                                              uint32_t *cols, uint64_t cols_cap);
/* Encode host columns as a stream in a new buffer (*ipc, *len; free with xlog_hip_bytes_free). */
xlog_hip_status xlog_hip_arrow_ipc_encode_u32(const uint32_t *const *cols, uint32_t arity, uint64_t rows,
                                              const char *const *names, uint8_t **ipc, uint64_t *len);
void xlog_hip_bytes_free(uint8_t *p);
/* Relation from a stream in host memory; each column buffer is copied once to
 * the device and packed there (reference: from_arrow_ipc_stream, provider/io.rs:716-739). */
xlog_hip_status xlog_hip_rel_from_arrow_ipc(xlog_hip_ctx *ctx, const uint8_t *ipc, uint64_t len, xlog_hip_rel **out);
/* Stream of a relation's columns (reference: to_arrow_ipc_stream, provider/io.rs:697-713). */
xlog_hip_status xlog_hip_rel_to_arrow_ipc(xlog_hip_ctx *ctx, const xlog_hip_rel *rel, const char *const *names,
                                          uint8_t **ipc, uint64_t *len);
/* File forms; the file is memory-mapped and its column buffers uploaded from
 * the mapping (reference: read_arrow_ipc_stream_file / write_arrow_ipc_stream_file,
 * provider/io.rs:743-772). */
xlog_hip_status xlog_hip_read_arrow_ipc_stream_file(xlog_hip_ctx *ctx, const char *path, xlog_hip_rel **out);
xlog_hip_status xlog_hip_write_arrow_ipc_stream_file(xlog_hip_ctx *ctx, const xlog_hip_rel *rel,
                                                     const char *const *names, const char *path);
/* Download column `col` into host[0..rows) (reference: download_column::<u32>, provider/transfer.rs:22). */
xlog_hip_status xlog_hip_rel_download_column(xlog_hip_ctx *ctx, const xlog_hip_rel *rel, uint32_t col,
                                             uint32_t *host, uint64_t host_cap);
/* Download packed keys of an arity<=2 relation into host[0..rows). */
xlog_hip_status xlog_hip_rel_download_packed(xlog_hip_ctx *ctx, const xlog_hip_rel *rel, uint64_t *host,
                                             uint64_t host_cap);
/* Logical row count (reference: device_row_count, provider/mod.rs:2823-2830). */
xlog_hip_status xlog_hip_rel_num_rows(const xlog_hip_rel *rel, uint64_t *rows);
xlog_hip_status xlog_hip_rel_arity(const xlog_hip_rel *rel, uint32_t *arity);
/* 1 if the relation is certified sorted by all columns and unique
 * (reference: the canonical-set certificate, memory.rs:1771-1773). */
xlog_hip_status xlog_hip_rel_is_canonical(const xlog_hip_rel *rel, int *canonical);
/* Device pointer to the packed key words (word 0 or 1) of a relation, for zero-copy consumers. */
xlog_hip_status xlog_hip_rel_device_words(const xlog_hip_rel *rel, uint32_t word, const uint64_t **dev);
/* Deep copy (reference: clone_buffer, relational.rs:6113). */
xlog_hip_status xlog_hip_rel_clone(xlog_hip_ctx *ctx, const xlog_hip_rel *in, xlog_hip_rel **out);
void xlog_hip_rel_free(xlog_hip_rel *rel);

/* ---- operators (CudaKernelProvider inherent methods) --------------------- */

/* Stable sort by key columns, listed most significant first; rows with equal
 * keys keep their input order (reference: sort, relational.rs:1881-2220). */
xlog_hip_status xlog_hip_sort(xlog_hip_ctx *ctx, const xlog_hip_rel *in, const uint32_t *key_cols,
                              uint32_t n_keys, xlog_hip_rel **out);
/* Keep the first row of every group of rows equal on key_cols, output sorted
 * by key_cols (reference: dedup, relational.rs:238-275). */
xlog_hip_status xlog_hip_dedup(xlog_hip_ctx *ctx, const xlog_hip_rel *in, const uint32_t *key_cols,
                               uint32_t n_keys, xlog_hip_rel **out);
/* Dedup of input already ordered on key_cols: the first row of every run of
 * adjacent rows equal on key_cols, input order, no sort; a full-row key list
 * on arity > 1 is the full-row dedup (reference: dedup_sorted, relational.rs:288-420). */
xlog_hip_status xlog_hip_dedup_sorted(xlog_hip_ctx *ctx, const xlog_hip_rel *in, const uint32_t *key_cols,
                                      uint32_t n_keys, xlog_hip_rel **out);
/* Full-row set: sort by every column, drop duplicate rows
 * (reference: dedup_full_row / dedup_full_row_deterministic, relational.rs:1458,1558-1677). */
xlog_hip_status xlog_hip_dedup_full_row(xlog_hip_ctx *ctx, const xlog_hip_rel *in, xlog_hip_rel **out);
/* Set union, canonical output (reference: union_gpu, relational.rs:822-824). */
xlog_hip_status xlog_hip_union(xlog_hip_ctx *ctx, const xlog_hip_rel *a, const xlog_hip_rel *b,
                               xlog_hip_rel **out);
/* Set union of many (reference: union_many_gpu, relational.rs:859-971). */
xlog_hip_status xlog_hip_union_many(xlog_hip_ctx *ctx, const xlog_hip_rel *const *ins, uint32_t n_ins,
                                    xlog_hip_rel **out);
/* Set difference dedup(a) \ b, canonical output
 * (reference: diff_gpu / diff_full_row, relational.rs:1102-1147,1489). */
xlog_hip_status xlog_hip_diff(xlog_hip_ctx *ctx, const xlog_hip_rel *a, const xlog_hip_rel *b,
                              xlog_hip_rel **out);
/* Equi-join on one key column per side.  INNER output = left columns ++
 * right columns (arity_l + arity_r <= 8), one row per matching pair, row
 * order unspecified (reference: hash_join_v2, relational.rs:2926-2992,4417-4625).
 * SEMI / ANTI output the left rows with / without a match. */
xlog_hip_status xlog_hip_hash_join(xlog_hip_ctx *ctx, const xlog_hip_rel *left, const xlog_hip_rel *right,
                                   uint32_t left_key, uint32_t right_key, int join_type, xlog_hip_rel **out);
/* Equi-join on n_keys key columns per side: left row i matches right row j
 * when left[i][left_keys[t]] == right[j][right_keys[t]] for every t
 * (reference: hash_join_v2(left, right, left_keys, right_keys, join_type),
 * relational.rs:2926-2992, keys packed by pack_and_hash_keys, pack.cu:144-214).
 * INNER output = left columns ++ right columns (arity_l + arity_r <= 8), rows
 * in left-row order and, per left row, right-row order; SEMI / ANTI output the
 * left rows with / without a match, in input order.  Each side holds fewer
 * than 2^32 - 1 rows (CAPACITY_OVERFLOW otherwise, as the reference's u32 row
 * indices). */
xlog_hip_status xlog_hip_hash_join_keys(xlog_hip_ctx *ctx, const xlog_hip_rel *left, const xlog_hip_rel *right,
                                        const uint32_t *left_keys, const uint32_t *right_keys, uint32_t n_keys,
                                        int join_type, xlog_hip_rel **out);
/* Join index over the key columns right_keys[0 .. n_keys) of `right`,
 * reused across probes (reference: build_join_index_v2(right, right_keys),
 * relational.rs:3728-3880, called with the rule's whole key list by the
 * executor's persistent-index join, node_dispatch.rs:444-488).  Fails on an
 * empty relation like the reference, and on one of 2^32 - 1 rows or more
 * (CAPACITY_OVERFLOW).  Free it with xlog_hip_join_index_free before its
 * context is destroyed. */
xlog_hip_status xlog_hip_join_index_build(xlog_hip_ctx *ctx, const xlog_hip_rel *right, const uint32_t *right_keys,
                                          uint32_t n_keys, xlog_hip_join_index **out);
/* xlog_hip_hash_join_keys against a prebuilt index of (right, right_keys);
 * the index must have been built over this right relation (same row count)
 * and exactly these right key columns, else INVALID_ARG
 * (reference: hash_join_v2_with_index, relational.rs:3882-4000).  The output
 * is that of xlog_hip_hash_join_keys: INNER rows left ++ right in left-row
 * order and, per left row, right-row order; max_output > 0 keeps the first
 * max_output INNER rows of that order (the reference keeps an unspecified
 * subset); SEMI / ANTI the left rows with / without a match. */
xlog_hip_status xlog_hip_hash_join_with_index(xlog_hip_ctx *ctx, const xlog_hip_rel *left, const xlog_hip_rel *right,
                                              const uint32_t *left_keys, const uint32_t *right_keys, uint32_t n_keys,
                                              int join_type, const xlog_hip_join_index *index, uint64_t max_output,
                                              xlog_hip_rel **out);
void xlog_hip_join_index_free(xlog_hip_join_index *index);
/* Nested-loop inner join on one key column, left ++ right columns, rows in
 * left-row-major then right-row order; CAPACITY_OVERFLOW when rows_l * rows_r
 * > 4,000,000 (reference: nested_loop_join_v2_inner_u32_1key,
 * relational.rs:3041-3255; NESTED_LOOP_TOTAL_THRESHOLD, provider/mod.rs:1030). */
xlog_hip_status xlog_hip_nested_loop_join(xlog_hip_ctx *ctx, const xlog_hip_rel *left, const xlog_hip_rel *right,
                                          uint32_t left_key, uint32_t right_key, xlog_hip_rel **out);
/* Sort-merge inner join on one u32 key column, left ++ right columns
 * (reference: sort_merge_join_v2_inner_u32_1key, relational.rs:3401-3728).
 * The reference requires both inputs sorted ascending on their key and at most
 * 4,000,000 row pairs; here an input whose key column is not sorted is sorted
 * first and there is no pair cap.  Left rows are matched to the right side's
 * runs of equal keys along the merge path; rows come out in left key order,
 * the right rows of a run in input order. */
xlog_hip_status xlog_hip_sort_merge_join(xlog_hip_ctx *ctx, const xlog_hip_rel *left, const xlog_hip_rel *right,
                                         uint32_t left_key, uint32_t right_key, xlog_hip_rel **out);
/* Fused join + projection: ChainJoin = Project(Join) (crates/xlog-logic/src/promote.rs:1020-1060,
 * expression.rs:779-834).  out_cols index the concatenated row (left ++ right);
 * the output has n_out (1 or 2) columns, bag semantics. */
xlog_hip_status xlog_hip_join_project(xlog_hip_ctx *ctx, const xlog_hip_rel *left, const xlog_hip_rel *right,
                                      uint32_t left_key, uint32_t right_key, const uint32_t *out_cols,
                                      uint32_t n_out, xlog_hip_rel **out);
/* Canonical set of the projected join: dedup_full_row(project(join(left, right))).
 * This is the ChainJoin -> Project -> dedup sequence of one rule contribution
 * (promote.rs:1020-1060, expression.rs:779-834, relational.rs:1558-1677) as one
 * operator; for output (left column, right non-key column) the join is emitted
 * in output order and the full sort of the join output is avoided. */
xlog_hip_status xlog_hip_join_project_dedup(xlog_hip_ctx *ctx, const xlog_hip_rel *left, const xlog_hip_rel *right,
                                            uint32_t left_key, uint32_t right_key, const uint32_t *out_cols,
                                            uint32_t n_out, xlog_hip_rel **out);
/* Column projection, bag semantics (reference: extract_column + combine_columns,
 * relational.rs:6196, provider/arithmetic.rs:1056). */
xlog_hip_status xlog_hip_project(xlog_hip_ctx *ctx, const xlog_hip_rel *in, const uint32_t *cols, uint32_t n_cols,
                                 xlog_hip_rel **out);
/* Non-decreasing check of one column (reference: is_sorted_ascending_u32, relational.rs:3258). */
xlog_hip_status xlog_hip_is_sorted(xlog_hip_ctx *ctx, const xlog_hip_rel *rel, uint32_t col, int *sorted);
/* In-place exclusive scan of a device u32 array; *total receives the sum
 * (reference: exclusive_scan_u32_inplace, provider/mod.rs:2177). */
xlog_hip_status xlog_hip_exclusive_scan_u32(xlog_hip_ctx *ctx, uint32_t *dev, uint64_t n, uint64_t *total);
/* xlog_hip_exclusive_scan_u32 without any device allocation.  No counterpart
 * in the reference: it is for callers that cannot allocate device memory
 * (tight serving loops, harnesses that forbid hipMalloc).  Its scratch
 * (ticket, total, look-back status) lives in a fixed device array of 2 MiB
 * per GPU, held from library load to process exit; n above 2^32 is
 * CAPACITY_OVERFLOW.  All calls on one GPU share that array: calls that
 * overlap on one GPU (two contexts on two threads) race.  It synchronises
 * the context stream to read *total, so it cannot be recorded into a HIP
 * graph (stream capture forbids the synchronisation). */
xlog_hip_status xlog_hip_exclusive_scan_u32_noalloc(xlog_hip_ctx *ctx, uint32_t *dev, uint64_t n, uint64_t *total);
/* Column roles of one factorized delta step (reference FjDeltaCols,
 * provider/fj_delta.rs:50-84); each pair is {0, 1} in some order. */
typedef struct {
    uint32_t delta_carry; /* delta column carried into the head */
    uint32_t delta_key;   /* delta column joined with edge column 0 */
    uint32_t r_carry;     /* head / full column holding the carry */
    uint32_t r_value;     /* head / full column holding edge column 1 */
} xlog_hip_fj_delta_cols;
/* One factorized semi-naive delta step over a dense domain:
 *   { head(carry, value) : delta(carry, key), edge(key, value), head not in full }
 * as a canonical (sorted, unique) arity-2 relation in full's column order.
 * Every id must be < domain and 0 < domain <= 2^16, else INVALID_ARG
 * (reference: fj_delta_novel_u32_recorded, provider/fj_delta.rs:117-490; the
 * reference's launch stream is the context's stream here). */
xlog_hip_status xlog_hip_fj_delta_novel(xlog_hip_ctx *ctx, const xlog_hip_rel *delta, const xlog_hip_rel *edge,
                                        const xlog_hip_rel *full, const xlog_hip_fj_delta_cols *cols,
                                        uint32_t domain, xlog_hip_rel **out);
/* The same step over a device hash set, with no domain bound (reference:
 * fj_delta_sparse_novel_u32_recorded, provider/fj_delta_sparse.rs:66).  The
 * table holds 2 x (|full| + candidate tuples) slots; when that is above
 * max_table_bytes (0: no budget) the call declines like the reference's
 * Ok(None): it returns XLOG_HIP_OK with *out = NULL.  The output is canonical
 * (the reference's is unordered). */
xlog_hip_status xlog_hip_fj_delta_sparse_novel(xlog_hip_ctx *ctx, const xlog_hip_rel *delta, const xlog_hip_rel *edge,
                                               const xlog_hip_rel *full, const xlog_hip_fj_delta_cols *cols,
                                               uint64_t max_table_bytes, xlog_hip_rel **out);
/* Keep rows whose device u8 mask is non-zero, input order
 * (reference: compact_buffer_by_device_mask_device_count, provider/filter.rs:1820-1935). */
xlog_hip_status xlog_hip_compact(xlog_hip_ctx *ctx, const xlog_hip_rel *in, const uint8_t *dev_mask,
                                 xlog_hip_rel **out);

/* ---- fixpoint driver (Executor::execute_recursive_scc, recursive.rs:447-957) ---- */

/* Program plan: int32 array
 *   [n_rules, then per rule: head_pred, hv0, hv1, n_body, (pred, v0, v1) * n_body]
 * over arity-2 predicates 0..n_preds-1; variables are small ints; 1..4 atoms
 * per body.  The join route evaluates bodies left-deep in body order: each
 * atom after the first shares one variable with the running binding, which
 * keeps at most two live variables, or both (a cyclic body such as a
 * triangle: the binding rows that form a row of the atom are kept), as the
 * reference's lowering joins on every shared variable (crates/xlog-logic/src/
 * lower.rs:1795-1850).  The bitmap route takes bodies whose atoms form a path from hv0
 * to hv1 in any order (each atom read forward or with its columns swapped).
 * rels[p] supplies every predicate (EDB facts; IDB initial contents, may be
 * empty).  On success out[p] receives a new canonical relation for every IDB
 * predicate (NULL for EDB ones).  Both routes give the same relations, the
 * same iteration count and the same per-iteration delta sizes. */
typedef struct {
    uint64_t iterations;      /* loop iterations incl. the final empty one (recursive.rs:619-620,860-865) */
    uint64_t max_iterations;  /* limit; 0 = 1,000,000 (config.rs:164) */
    uint64_t *delta_sizes;    /* optional: [0] seed delta, [k] total |delta| after iteration k */
    uint64_t delta_cap;       /* entries available in delta_sizes */
    uint64_t route;           /* XLOG_HIP_ROUTE_* (in: request, out: taken) */
    double wall_ms;           /* device wall time of the fixpoint */
    uint64_t max_join_rows;   /* in: 0 = no limit; otherwise a binary join of a rule body whose output
                                 (a bag) would exceed it fails with CAPACITY_OVERFLOW before it is
                                 materialised.  4294967295 reproduces the reference's u32 join-row
                                 limit (relational.rs:4550-4555). */
    uint64_t host_waits;      /* out: times the host waited for the device during the fixpoint
                                 (each count or size read-back is one wait) */
    uint64_t delta_count;     /* out: entries of delta_sizes written (the seed and each completed iteration);
                                 after a failure inside an iteration, iterations counts that iteration
                                 and delta_count - 1 the ones completed before it */
} xlog_hip_fixpoint_stats;

/* AUTO takes the bitmap route when every rule body is a path, there are at
 * most 2^17 distinct ids (max id + 1) and the bit matrices fit in half the
 * free device memory; otherwise the hash route when every rule body is a path
 * of at most three atoms, no join-row limit is set and no three-atom body
 * reads two IDB atoms; the join route otherwise.  Requesting BITMAP or HASH
 * for a plan or domain it cannot take is UNSUPPORTED. */
#define XLOG_HIP_ROUTE_AUTO 0
#define XLOG_HIP_ROUTE_JOIN 1   /* join -> sort -> dedup -> diff -> merge */
#define XLOG_HIP_ROUTE_BITMAP 2 /* relations as domain x domain bit matrices, rule bodies as chains of
                                   boolean products (the dense factorized delta of provider/fj_delta.rs:117
                                   generalised from transitive closure to path-shaped bodies) */
#define XLOG_HIP_ROUTE_HASH 3   /* every IDB relation also in a device hash set; each rule variant is one
                                   fused pass that expands the delta rows through the other atoms' run
                                   indexes (up to two hops, no intermediate relation: the multiway path
                                   join) and inserts the head tuples, the inserted ones being the next
                                   delta (the sparse factorized delta of provider/fj_delta_sparse.rs:66
                                   with a persistent table); bodies of 1 to 3 atoms forming a path.
                                   Programs whose variants read no IDB relation in full (linear ones)
                                   queue up to 8 iterations per host read-back */

xlog_hip_status xlog_hip_fixpoint(xlog_hip_ctx *ctx, const int32_t *plan, uint32_t n_preds,
                                  const xlog_hip_rel *const *rels, xlog_hip_rel **out,
                                  xlog_hip_fixpoint_stats *stats);

/* Transitive closure reach(X,Y) :- edge(X,Y). reach(X,Z) :- reach(X,Y), edge(Y,Z).
 * Convenience over xlog_hip_fixpoint with the TC plan. */
xlog_hip_status xlog_hip_fixpoint_tc(xlog_hip_ctx *ctx, const xlog_hip_rel *edge, xlog_hip_rel **reach,
                                     xlog_hip_fixpoint_stats *stats);

/* ---- kernel timing (diagnostics; no counterpart in the reference) ---------
 * With profiling enabled every launch of the listed kernel kinds is bracketed
 * by HIP events on the context stream.  profile_read synchronises and returns
 * the number of launches, their summed duration and summed algorithmic bytes
 * (the compulsory HBM bytes of the operation, e.g. 16 B per key per radix pass). */
#define XLOG_HIP_KERNEL_SORT_PASS 0   /* onesweep digit pass */
#define XLOG_HIP_KERNEL_SORT_HIST 1   /* 8-digit histogram */
#define XLOG_HIP_KERNEL_SELECT 2      /* dedup / diff / compaction */
#define XLOG_HIP_KERNEL_MERGE 3       /* merge-path merge */
#define XLOG_HIP_KERNEL_PROBE_COUNT 4 /* join probe, count pass */
#define XLOG_HIP_KERNEL_PROBE_EMIT 5  /* join probe, materialise pass */
#define XLOG_HIP_KERNEL_TC_STEP 6     /* dense TC iteration */
#define XLOG_HIP_KERNEL_TC_EMIT 7     /* dense TC final emit */
#define XLOG_HIP_KERNEL_CHAIN_PRODUCT 8  /* dense chain-rule boolean product */
#define XLOG_HIP_KERNEL_CHAIN_FINALIZE 9 /* dense chain-rule delta / merge */
#define XLOG_HIP_KERNEL_CHAIN_EMIT 10    /* dense chain-rule final emit */
#define XLOG_HIP_KERNEL_HASH_INSERT 11   /* sparse delta step: expand + hash-set insert */
#define XLOG_HIP_KERNEL_SORT_RUNS 12     /* sort of short runs by the low word */
#define XLOG_HIP_KERNEL_SORT_SEGMENTS 13 /* on-chip sort of top-16-bit segments */
#define XLOG_HIP_KERNEL_KINDS 14
xlog_hip_status xlog_hip_profile_enable(xlog_hip_ctx *ctx, int on);
xlog_hip_status xlog_hip_profile_reset(xlog_hip_ctx *ctx);
xlog_hip_status xlog_hip_profile_read(xlog_hip_ctx *ctx, uint32_t kind, uint64_t *launches, double *total_ms,
                                      double *algo_bytes);

/* FNV-1a-64 over the little-endian bytes of the packed keys in row order
 * (offset / prime as kernels/pack.cu:8-9); host-side, downloads the relation. */
xlog_hip_status xlog_hip_rel_digest(xlog_hip_ctx *ctx, const xlog_hip_rel *rel, uint64_t *digest);

#ifdef __cplusplus
}
#endif
#endif /* XLOG_HIP_H */
