/*
 * lsa_rocm.h - C ABI of the MI355X (gfx950) select+read kernels for Latent Sparse
 * Attention. One shared library, liblsa_rocm.so; every entry point:
 *   - takes plain device pointers, sizes and a hipStream_t (as void*); the library
 *     never allocates device memory: scratch comes in through `workspace`;
 *   - launches asynchronously on that stream and never synchronizes;
 *   - validates its arguments on the host first and returns LSA_OK (0) or a negative
 *     LSA_ERR_* code, with a message from lsa_last_error() (thread-local).
 * Layouts are dense row-major (the Python host layer makes tensors contiguous).
 *
 * Selection keys are the reference's packed int64 layout:
 *   key = (ordered_bits(score) << 32) | (0x7FFFFFFF - column),  EMPTY = INT64_MIN.
 * Scores are the canonical fp32 dot product: operands rounded to the scoring type
 * (bf16 RNE or fp32), exact fp64 products, 16 in-order partial sums over contiguous
 * D/16 slices, combined by the tree (p,p+8),(p,p+4),(p,p+2),(p,p+1), one fp32 rounding.
 *
 * Bucket tables: a contiguous stack of `n_tables` tables, each `rows` buckets. The
 * table used by (query row r, group g) is r * row_tables + g * group_tables, so
 * (0, 0) shares one table (the reference layout), (0, 1) is one table per kv-head
 * (per-kv-head selection) and (G, 1) one per (sequence, kv-head).
 */
#ifndef LSA_ROCM_H
#define LSA_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LSA_ABI_VERSION 3

enum lsa_status {
  LSA_OK = 0,
  LSA_ERR_NULL = -1,      /* a required pointer is NULL */
  LSA_ERR_SHAPE = -2,     /* sizes inconsistent or out of the supported range */
  LSA_ERR_DTYPE = -3,     /* unsupported element type */
  LSA_ERR_POW2 = -4,      /* a size that must be a power of two is not */
  LSA_ERR_WORKSPACE = -5, /* workspace missing or too small */
  LSA_ERR_LAUNCH = -6,    /* the HIP launch failed */
  LSA_ERR_ALIGN = -7      /* a pointer is not aligned for vector access */
};

enum lsa_dtype { LSA_F32 = 0, LSA_BF16 = 1, LSA_F16 = 2 };
enum lsa_score_mode { LSA_SCORE_BF16 = 0, LSA_SCORE_F32 = 1 };
enum lsa_centroid_mode { LSA_CENTROID_MEAN = 0, LSA_CENTROID_NORMALIZED = 1, LSA_CENTROID_SUM = 2 };

/* A paged K/V cache's slot table (upstream's paged decode: the reference's expansion kernel
 * maps every kept id and the window/sink tail through a slot table, select_fused.py:147-205
 * `slot_table_ptr` / `slot_rows_ptr` / `MAP_SLOTS`). Logical position p of query row r lives
 * in physical cache row table[rows[r] * stride + p]. The selects and the fused decode apply
 * the map where they write a read list - once per listed id - so lists hold physical rows
 * and the gather reads them with no extra load; which ids are kept (sink <= id < window
 * start, top_k) is decided on the logical positions, as the reference does. The chunked
 * prefill read maps its causal block the same way (its chunk lists are already physical).
 * Passed as `const lsa_slot_map*`; NULL means ids are cache rows (no paging). */
typedef struct lsa_slot_map {
  const int32_t* table; /* [n_rows, stride] int32 physical cache rows (-1: no row) */
  const int32_t* rows;  /* [R] int32: the table row of each query row (decode: batch row) */
  int64_t stride;       /* elements between table rows, >= width */
  int32_t width;        /* logical positions a table row maps (>= 1); ids at or past it map to -1 */
  int32_t n_rows;       /* table rows; a row index outside [0, n_rows) maps every id to -1 */
} lsa_slot_map;

int lsa_abi_version(void);
const char* lsa_last_error(void);

/* Visible bucket counts per (row, group) [R, G] int32 (reference pipeline.py:184-186
 * visible_counts): without `ends`, (pos // cluster_block_size) * block_buckets clamped
 * to rows; with `ends` [tables, rows] the buckets whose span ends at or before pos+1. */
int lsa_visible_counts(const int32_t* positions, int64_t R, int32_t G, int32_t rows, int32_t cluster_block_size,
                       int32_t block_buckets, const int32_t* ends, int64_t row_tables, int64_t group_tables,
                       int32_t* counts, void* stream);

/* Canonical scores [R, G, N] fp32 of queries [R, G, D] (dtype q_dtype) against the
 * tables' centroids (bf16 for LSA_SCORE_BF16, fp32 for LSA_SCORE_F32). Replaces the
 * reference's score GEMM, pipeline.py:217-232 _production_scores. */
int lsa_score_rows(const void* queries, int q_dtype, int64_t R, int32_t G, int32_t D, const void* centroids,
                   int32_t N, int64_t row_tables, int64_t group_tables, int score_mode, float* scores, void* stream);

/* Whole-path listing: keys [R, N] int64, every column packed, EMPTY at or past
 * counts[r] (reference pipeline.py:266-267, upstream TopK.listed whole path). */
int lsa_pack_listing(const float* scores, const int32_t* counts, int64_t R, int32_t N, int64_t* keys, void* stream);

/* best_first_keys (reference pipeline.py:189-214): out [R, k] the k greatest keys of
 * each row of keys [R, W], descending; counts (nullable) masks slots >= counts[r]. */
int lsa_topk_keys(const int64_t* keys, const int32_t* counts, int64_t R, int32_t W, int32_t k, int64_t* out,
                  void* stream);

/* select_topk_scores (reference select_fused.py:83-137): out [R, K2] int64 with
 * K2 = next_pow2(min(top_p, N)), the best min(top_p, N) packed keys of the fp32 scores
 * [R, N] (columns >= lengths[r] are EMPTY), descending, EMPTY tail. */
int lsa_select_topk_scores(const float* scores, const int32_t* lengths, int64_t R, int32_t N, int32_t top_p,
                           int64_t* out, void* stream);

/* unpack_ids (upstream keys.unpack_ids, reference pipeline.py:268): ids [n] int32. */
int lsa_unpack_ids(const int64_t* keys, int64_t n, int32_t* ids, void* stream);

/* Rank-order expansion (upstream expand_in_order, reference select_fused.py:140-280
 * expand_in_order_from_keys). picks [R, G, P]: int32 bucket ids (-1 none) when
 * picks_are_keys == 0, int64 packed keys (EMPTY none) otherwise. members [tables, rows,
 * cap]; positions [R] int32. Out: lists [R, G, top_k + window + sink] int32 (-1 padded)
 * and lengths [R, G] int32. */
int lsa_expand(const void* picks, int picks_are_keys, int64_t R, int32_t G, int32_t P, const int32_t* members,
               int32_t rows, int32_t cap, int64_t row_tables, int64_t group_tables, const int32_t* positions,
               const lsa_slot_map* slots, int32_t window, int32_t sink, int32_t top_k, int32_t* lists,
               int32_t* lengths, void* stream);

/* Fused flat select: score + top-k + expansion in one launch (reference pipeline.py:
 * 274-316 flat_select, LSA_SELECT_IMPL=fused). queries [R, G, D]; tables as above
 * (centroids bf16 or fp32 per score_mode, members, optional ends); positions [R]. The
 * N columns of a (row, group) are split over `splits` workgroups whose sorted partial
 * top-k lists the last one to arrive merges (splits == 1: counters and scratch unused).
 * counters: R * G int32 that read zero at launch; every launch leaves them zero again.
 * scratch: lsa_select_flat_scratch_bytes(), no initialisation. table_flags: 0 or
 * LSA_TABLE_SPANS (span tables: with at most 4096 picks the expansion takes each pick's
 * kept ids from the span ends, with no member-row loads; the lists are the ones the member
 * rows give), optionally with LSA_TABLE_BLOCK_VISIBLE. Out as lsa_expand. */
size_t lsa_select_flat_scratch_bytes(int64_t R, int32_t G, int32_t top_p, int32_t N, int32_t splits);
int lsa_select_flat(const void* queries, int q_dtype, int64_t R, int32_t G, int32_t D, const void* centroids,
                    const int32_t* members, const int32_t* ends, int32_t table_flags, int32_t rows, int32_t cap,
                    int64_t row_tables,
                    int64_t group_tables, int score_mode, const int32_t* positions, const lsa_slot_map* slots,
                    int32_t cluster_block_size, int32_t block_buckets, int32_t top_p, int32_t window, int32_t sink,
                    int32_t top_k, int32_t splits, int32_t* counters, void* scratch, size_t scratch_bytes,
                    int32_t* lists, int32_t* lengths, void* stream);

/* Two-level tree select (reference pipeline.py:319-337 tree_select, _tree.py:318-373
 * _beam_pick_rows with one node level, _tree.py:100-142 _growth_replay): per (row, group)
 * with V visible buckets, node growth covers the first C = min(floor(V / node_block) *
 * node_block, n_nodes * node_size) buckets (node_block = the reference's
 * node_cluster_block_size), so the made nodes are [0, C / node_size). The best
 * `beam_width` made nodes (a tie to the lower node), then the best top_p of their visible
 * children plus the fresh buckets [C, V), each bucket once (a tie to the lower bucket),
 * then the flat expansion. node_centroids [tables, n_nodes, D], children [tables,
 * n_nodes, node_size] int32 bucket ids (node n's children lie in [0, (n + 1) * node_size),
 * as growth makes them). table_flags as lsa_select_flat. */
int lsa_select_tree(const void* queries, int q_dtype, int64_t R, int32_t G, int32_t D, const void* node_centroids,
                    const int32_t* children, int32_t n_nodes, int32_t node_size, const void* centroids,
                    const int32_t* members, const int32_t* ends, int32_t table_flags, int32_t rows, int32_t cap, int64_t row_tables,
                    int64_t group_tables, int score_mode, const int32_t* positions, const lsa_slot_map* slots,
                    int32_t cluster_block_size, int32_t block_buckets, int32_t node_block, int32_t beam_width,
                    int32_t top_p, int32_t window, int32_t sink, int32_t top_k, int32_t* lists, int32_t* lengths,
                    void* stream);

/* Multi-level beam select (reference pipeline.py:319-337 tree_select over a hierarchy of
 * several node levels: _tree.py:318-373 _beam_pick_rows, _tree.py:306-315 _dedup_scores,
 * with the growth of _tree.py:100-142 _growth_replay at page end V = the row's visible
 * bucket count). Level l + 1 (l = 0 .. n_levels - 1, bottom up) has n_nodes[l] nodes:
 * node_centroids[l] [tables, n_nodes[l], D] (bf16 or fp32 as score_mode), children[l]
 * [tables, n_nodes[l], node_size] int32 rows of the level below (bucket rows for l = 0).
 * Growth: covered C = floor(V / node_block) * node_block buckets make C / node_size level-1
 * nodes; a level's nodes close in whole node_block blocks, closed / node_size nodes of the
 * level above being made, for min(n_levels, top_level) levels, each capped by n_nodes. The
 * walk starts at the highest level with a made node (all its made nodes are candidates);
 * below, the carried children plus the level's open nodes [closed, made); at the buckets
 * the carried children below V plus the fresh buckets [C, V). Each level scores each
 * candidate once and keeps the best beam_width (top_p at the buckets), a tie to the lower
 * row; then the flat expansion. Unlike the reference's torch walk, fewer candidates than
 * top_p leave -1 picks (its tail repeats -inf-scored candidates). Limits: n_levels <=
 * LSA_BEAM_MAX_LEVELS, rows and n_nodes[l] <= 8192, at most 4096 candidates a level.
 * table_flags as lsa_select_flat. */
#define LSA_BEAM_MAX_LEVELS 4
int lsa_select_beam(const void* queries, int q_dtype, int64_t R, int32_t G, int32_t D, int32_t n_levels,
                    const void* const* node_centroids, const int32_t* const* children, const int32_t* n_nodes,
                    int32_t node_size, int32_t node_block, int32_t top_level, const void* centroids,
                    const int32_t* members, const int32_t* ends, int32_t table_flags, int32_t rows, int32_t cap,
                    int64_t row_tables, int64_t group_tables, int score_mode, const int32_t* positions,
                    const lsa_slot_map* slots, int32_t cluster_block_size, int32_t block_buckets,
                    int32_t beam_width, int32_t top_p, int32_t window, int32_t sink, int32_t top_k, int32_t* lists,
                    int32_t* lengths, void* stream);

/* GQA-collapsed index queries (reference gates.py:50-59 make_index_space, per-kv-head
 * form): out [B, T/chunk, Hkv, D] fp32 = fp32 mean of q [B, T, Hq, D] over each
 * kv-head's query group and `chunk` consecutive tokens (tokens outer, heads inner). */
int lsa_index_queries(const void* q, int q_dtype, int64_t B, int64_t T, int32_t Hq, int32_t Hkv, int32_t D,
                      int32_t chunk, float* out, void* stream);

/* Bucket centroids (reference pipeline.py:108-115, :396-403): for each of n_tables *
 * rows buckets, the mean, the L2-normalized sum or the sum (the hierarchy's key sums,
 * reference pipeline.py:163-164) of its member keys. keys: element
 * (t, d) of table k lives at keys[k_off(k) + t * token_stride + d] with k_off(k) =
 * (k / kv_heads) * batch_stride + (k % kv_heads) * D; member ids outside [0, tokens) are
 * skipped. Out fp32 and bf16 [tables, rows, D]. */
int lsa_bucket_centroids(const void* keys, int k_dtype, int64_t tokens, int64_t token_stride, int64_t batch_stride,
                         int32_t kv_heads, int32_t D, const int32_t* members, int64_t n_tables, int32_t rows,
                         int32_t cap, int centroid_mode, float* out_f32, uint16_t* out_bf16, void* stream);

/* Bucket-table build from the keys (the index build before the path; replaces the
 * reference's build_buckets_gpu, pipeline.py:71-116, with contiguous segments): per table
 * (batch b, kv-head g) the keys [T, D] at keys + b * kv_sb + g * kv_sh + t * kv_st + d are
 * cut into pools of `pool` positions (fp64 sums), then the adjacent pair with the smallest
 * Ward cost n_a n_b / (n_a + n_b) |mu_a - mu_b|^2 is merged (ties to the leftmost pair,
 * merges past max_size positions skipped) until `target` segments remain. starts
 * [B * Hkv, target + 1] int32 receives each table's segment start positions (last = T);
 * status [B * Hkv] int32 receives 0, or 1 where no pair could merge before the target
 * (that table's starts are then the even cut floor(j * T / target), so every later kernel
 * reads valid positions). failed (nullable; device or pinned host memory) is set to 1 with
 * a system-scope store when any table fails, so a caller learns of it without a device sync
 * (it is never cleared here). scratch: lsa_ward_segments_scratch_bytes bytes of device
 * memory. Limits: ceil(T / pool) <= 4096 pools, target <= pools, max_size >= pool,
 * D <= 1024. */
size_t lsa_ward_segments_scratch_bytes(int64_t tables, int64_t T, int32_t D, int32_t pool);
int lsa_ward_segments(const void* keys, int k_dtype, int64_t B, int64_t T, int32_t kv_heads, int32_t D,
                      int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int32_t pool, int32_t target, int32_t max_size,
                      void* scratch, size_t scratch_bytes, int32_t* starts, int32_t* status, int32_t* failed,
                      void* stream);

/* Sparse gather read (reference read_kernel_tiled.py:30-156 sparse_read_auto / tiled,
 * read_kernel.py:26-120 v1): q [B, Tq, Hq, D] dense; k/v [B, Tk, Hkv, D] (dtype) with the
 * given element strides of batch, token and head (shared by K and V; rows of D contiguous
 * elements, 16-byte aligned), so a view into a larger cache is read in place; ids
 * [B*Tq, W] shared by all heads (ids_per_head == 0) or [B*Tq, Hkv, W] per kv-head, and
 * lengths likewise. Each (row, kv-head) list is cut into spans of whole tiles, at most
 * `splits` (<= 256) of them; the online-softmax partials of a row's active spans are
 * combined by the last workgroup to arrive. empty_nan: a row with no key
 * gives NaN (v1 contract) instead of 0. Ids outside [0, Tk) are skipped.
 * counters: B*Tq*Hkv int32 that read zero at launch, left zero (splits > 1 only);
 * scratch: lsa_read_scratch_bytes(), no initialisation. */
size_t lsa_read_scratch_bytes(int64_t rows, int32_t Hq, int32_t Hkv, int32_t D, int32_t splits);
/* List slots one read workgroup covers per tile for (dtype, head dim, query heads per
 * kv-head); a split spans ceil(ceil(W / tile) / splits) tiles. 0 for unsupported dims. */
int32_t lsa_read_tile_tokens(int dtype, int32_t D, int32_t group);
int lsa_read(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t Tq, int64_t Tk, int32_t Hq,
             int32_t Hkv, int32_t D, int64_t kv_batch_stride, int64_t kv_token_stride, int64_t kv_head_stride,
             const int32_t* ids, const int32_t* lengths, int32_t W, int ids_per_head, float scale, int empty_nan,
             int32_t splits, int32_t* counters, void* scratch, size_t scratch_bytes, void* out, void* stream);

/* Chunked prefill read: query row t of chunk c = t / chunk reads chunk c's per-kv-head
 * list ids [B, C, Hkv, W] (first lengths[b, c, g] slots) plus the chunk's causal block
 * [c*chunk, t]. q [B, T, Hq, D], k/v [B, Tk, Hkv, D], out like q; T <= Tk.
 * path: LSA_CHUNKED_AUTO (the MFMA tile kernel when lsa_read_chunked_mfma_ok, else the
 * gather kernel), LSA_CHUNKED_GATHER, or LSA_CHUNKED_MFMA (an error where it does not
 * apply). */
#define LSA_CHUNKED_AUTO 0
#define LSA_CHUNKED_GATHER 1
#define LSA_CHUNKED_MFMA 2
int lsa_read_chunked(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t T, int64_t Tk,
                     int32_t Hq, int32_t Hkv, int32_t D, int64_t kv_batch_stride, int64_t kv_token_stride,
                     int64_t kv_head_stride, const int32_t* ids, const int32_t* lengths, int32_t W, int32_t chunk,
                     const lsa_slot_map* slots, float scale, int32_t path, void* out, void* stream);
/* 1 when the MFMA tile kernel serves lsa_read_chunked for this shape: bf16/fp16 rows, head
 * dim 64 or 128, chunk in {16, 32, 64, 128, 256}. */
int lsa_read_chunked_mfma_ok(int dtype, int32_t D, int32_t chunk);

/* Fused decode step: the flat select and the sparse read of one decode token per batch
 * row in ONE launch (reference port/bench.py:147-153 `step` = pipeline.flat_select then
 * read_kernel_tiled.sparse_read_auto; pipeline.py:248-316, select_fused.py:52-280,
 * read_kernel_tiled.py:92-156). Row r's index query is the fp32 mean of its query group
 * (make_index_space, gates.py:50-59). q [R, Hq, D] (one token per batch row), k/v
 * [R, Tk, Hkv, D] at the given element strides, tables as lsa_select_flat's; writes
 * lists [R, Hkv, top_k + window + sink] and lengths [R, Hkv] (identical to
 * lsa_select_flat's) and out [R, Hq, D] (the read of those lists).
 *
 * select_splits: select workgroups per (row, kv-head), 1..min(256, rows) (the exchange
 * form: the splits score slices of the table and the last to arrive publishes the picks
 * to the readers), or 0: the replicated form, with no select workgroups - every reader
 * workgroup scores its unit's whole table (a matrix-core screen with a proven error
 * bound, then the exact canonical score of the few rows near the cut), so no workgroup
 * waits on another before the gather; the picks and lists are the same. The replicated
 * form needs LSA_TABLE_SPANS, bf16 scoring, head dim <= 128, at most 1024 buckets and 64
 * picks (lsa_decode_flat_rep_ok).
 * readers: reader workgroups per (row, kv-head), 0 = default (picks + the window/sink
 * parts), at most 256; each reads its share of the list in tiles of
 * lsa_read_tile_tokens() slots. counters: lsa_decode_flat_counters() int32 words, zero
 * before the first launch; every launch leaves them zero. scratch:
 * lsa_decode_flat_scratch_bytes(), 16-byte aligned. Launches sharing counters must be
 * stream-ordered. status (optional, int32 in device or pinned host memory; written with a
 * system-scope store) is set to 1 if a reader workgroup gave up waiting for its unit's
 * selection (not expected: readers wait only on lower-numbered workgroups, which never
 * wait). Such a reader writes nothing and still arrives, so the arrival counters reset,
 * but that launch's outputs are invalid and a record (or published keys) written after the
 * give-up can outlive it: the caller zeroes the counters before the next launch. With
 * more than one select split and a table that fits the counters' key slots (at most 1024
 * buckets, 65 536 (row, kv-head, bucket) slots in all), the splits publish their keys and
 * every reader ranks them itself (the rank form: the same lists).
 * table_flags: 0, or LSA_TABLE_SPANS when every bucket row j holds exactly the consecutive
 * ids ends[j - 1] .. ends[j] - 1 (ends[-1] = 0) in order, -1 after (the contiguous-segment
 * tables): the kept members of a pick are then a range, counted and expanded without
 * reading the member rows (the same lists). Requires ends.
 * Limits: top_p (capped at rows) <= 64; head dim {32,64,128,256}; group {1,2,4,8}. */
#define LSA_TABLE_SPANS 1
/* Table flag (every select and decode entry): visibility by the closed-block rule (pos //
 * cluster_block_size * block_buckets), as for tables without ends, while the ends serve the
 * span expansion only. Positional block tables (reference pipeline.py:378-403) are spans,
 * but a block is visible only once closed (pipeline.py:184-186), not when its span ends. */
#define LSA_TABLE_BLOCK_VISIBLE 2
int64_t lsa_decode_flat_counters(int64_t R, int32_t Hkv, int32_t rows, int32_t top_p);
/* 1 when lsa_decode_flat's replicated form (select_splits 0) serves this shape. */
int lsa_decode_flat_rep_ok(int dtype, int32_t D, int32_t group, int32_t rows, int32_t top_p, int score_mode,
                           int32_t table_flags);
size_t lsa_decode_flat_scratch_bytes(int dtype, int64_t R, int32_t Hq, int32_t Hkv, int32_t D, int32_t rows,
                                     int32_t top_p, int32_t window, int32_t sink, int32_t select_splits,
                                     int32_t readers);
int lsa_decode_flat(const void* q, const void* k, const void* v, int dtype, int64_t R, int64_t Tk, int32_t Hq,
                    int32_t Hkv, int32_t D, int64_t kv_batch_stride, int64_t kv_token_stride, int64_t kv_head_stride,
                    const void* centroids, const int32_t* members, const int32_t* ends, int32_t table_flags,
                    int32_t rows, int32_t cap,
                    int64_t row_tables, int64_t group_tables, int score_mode, const int32_t* positions,
                    const lsa_slot_map* slots, int32_t cluster_block_size, int32_t block_buckets, int32_t top_p,
                    int32_t window, int32_t sink, int32_t top_k, float scale, int32_t select_splits,
                    int32_t readers, int32_t* counters, int64_t n_counters, void* scratch, size_t scratch_bytes,
                    int32_t* lists, int32_t* lengths, void* out, int32_t* status, void* stream);

/* The fused decode step over a one-level node tree (reference port/bench.py:147-153 with
 * tree_select for flat_select: pipeline.py:319-337, _tree.py:318-373 with one node level,
 * the growth of _tree.py:100-142): one launch holds one select workgroup per (row,
 * kv-head) - the group-mean index query, the made nodes' best beam_width, then the best
 * top_p of their visible children plus the fresh buckets, exactly lsa_select_tree's lists -
 * and the readers of lsa_decode_flat. node_centroids [tables, n_nodes, D] in the scoring
 * type, children [tables, n_nodes, node_size] int32 bucket rows; at most 64 picks and 8192
 * buckets a table. Counters and scratch as lsa_decode_flat with one select split
 * (lsa_decode_flat_counters, lsa_decode_flat_scratch_bytes(..., select_splits = 1, ...)). */
int lsa_decode_tree(const void* q, const void* k, const void* v, int dtype, int64_t R, int64_t Tk, int32_t Hq,
                    int32_t Hkv, int32_t D, int64_t kv_batch_stride, int64_t kv_token_stride, int64_t kv_head_stride,
                    const void* node_centroids, const int32_t* children, int32_t n_nodes, int32_t node_size,
                    int32_t node_block, int32_t beam_width, const void* centroids, const int32_t* members,
                    const int32_t* ends, int32_t table_flags, int32_t rows, int32_t cap, int64_t row_tables,
                    int64_t group_tables, int score_mode, const int32_t* positions, const lsa_slot_map* slots,
                    int32_t cluster_block_size, int32_t block_buckets, int32_t top_p, int32_t window, int32_t sink,
                    int32_t top_k, float scale, int32_t readers, int32_t* counters, int64_t n_counters,
                    void* scratch, size_t scratch_bytes, int32_t* lists, int32_t* lengths, void* out,
                    int32_t* status, void* stream);

/* Fused decode step over the reference's own layout - one index-space selection a query row
 * shared by every kv-head (reference port/bench.py:147-153 `step` = pipeline.py:248-316
 * flat_select on the index space, then read_kernel_tiled.py:92-156 over [B, Tq, W] lists
 * shared by the heads) - at its own knobs (PortConfig, pipeline.py:32-54: up to 4096
 * buckets, top_p 1024, top_k 4096). index_queries [R, D] fp32 (one a row: the reference's
 * make_index_space output); one span table a row (row_tables 1) or for every row (0):
 * centroids [tables, rows, D] (bf16 or fp32 per score_mode) and span ends [tables, rows]
 * (LSA_TABLE_SPANS required, LSA_TABLE_BLOCK_VISIBLE optional). q [R, Hq, D], k/v as
 * lsa_decode_flat's (bf16 or fp16, head dim 64 or 128). Writes lists [R, top_k + window +
 * sink] and lengths [R] (identical to lsa_select_flat's on the same queries and table) and
 * out [R, Hq, D] (the read of those lists). select_splits: select workgroups a row (0 = one
 * a 64 buckets, at most 256); readers: reader workgroups a (row, kv-head) (0 = default, at
 * most 64). counters: lsa_decode_shared_counters() int32 words (8-byte aligned), zero before
 * the first launch; every launch leaves them zero. scratch: lsa_decode_shared_scratch_bytes().
 * status as lsa_decode_flat's. Limits: at most 4096 buckets and 1024 picks a row, the
 * reader LDS within 64 KiB. */
int64_t lsa_decode_shared_counters(int64_t R, int32_t Hkv, int32_t rows);
size_t lsa_decode_shared_scratch_bytes(int dtype, int64_t R, int32_t Hq, int32_t Hkv, int32_t D, int32_t rows,
                                       int32_t top_p, int32_t window, int32_t sink, int32_t top_k, int32_t readers);
int lsa_decode_shared(const void* q, const void* k, const void* v, int dtype, int64_t R, int64_t Tk, int32_t Hq,
                      int32_t Hkv, int32_t D, int64_t kv_batch_stride, int64_t kv_token_stride, int64_t kv_head_stride,
                      const float* index_queries, const void* centroids, const int32_t* ends, int32_t table_flags,
                      int32_t rows, int64_t row_tables, int score_mode, const int32_t* positions,
                      const lsa_slot_map* slots, int32_t cluster_block_size, int32_t block_buckets, int32_t top_p,
                      int32_t window, int32_t sink, int32_t top_k, float scale, int32_t select_splits,
                      int32_t readers, int32_t* counters, int64_t n_counters, void* scratch, size_t scratch_bytes,
                      int32_t* lists, int32_t* lengths, void* out, int32_t* status, void* stream);

/* lsa_decode_shared with the tree arm's selection: one multi-level beam walk a query row over
 * the index-space hierarchy, shared by every kv-head (reference port/bench.py:147-153 `step`
 * with tree_select = pipeline.py:319-337 over the index space, then read_kernel_tiled.py:
 * 92-156 over [B, Tq, W] lists), at its own knobs (PortConfig: node size 4, node blocks of
 * 64, 3 levels, beam 64, top_p 1024). Levels, children, growth and candidate rules as
 * lsa_select_beam (n_levels, node_centroids, children, n_nodes, node_size, node_block,
 * top_level, beam_width); one table a row (row_tables 1) or for every row (0), span ends
 * required (LSA_TABLE_SPANS, optionally LSA_TABLE_BLOCK_VISIBLE); the other arguments as
 * lsa_decode_shared. Lists and lengths are identical to lsa_select_beam's on the same
 * queries and tables; out is the read of those lists. counters:
 * lsa_decode_tree_shared_counters() int32 words (8-byte aligned), zero before the first
 * launch, left zero; scratch: lsa_decode_shared_scratch_bytes(). Limits: rows and
 * n_nodes[l] <= 8192, at most 4096 candidates a level, min(top_p, candidates) <= 1024
 * picks, the reader LDS within 64 KiB. */
int64_t lsa_decode_tree_shared_counters(int64_t R, int32_t Hkv, int32_t n_levels, const int32_t* n_nodes,
                                        int32_t rows);
int lsa_decode_tree_shared(const void* q, const void* k, const void* v, int dtype, int64_t R, int64_t Tk, int32_t Hq,
                           int32_t Hkv, int32_t D, int64_t kv_batch_stride, int64_t kv_token_stride,
                           int64_t kv_head_stride, const float* index_queries, int32_t n_levels,
                           const void* const* node_centroids, const int32_t* const* children,
                           const int32_t* n_nodes, int32_t node_size, int32_t node_block, int32_t top_level,
                           const void* centroids, const int32_t* ends, int32_t table_flags, int32_t rows,
                           int64_t row_tables, int score_mode, const int32_t* positions,
                           const lsa_slot_map* slots, int32_t cluster_block_size, int32_t block_buckets,
                           int32_t beam_width, int32_t top_p, int32_t window, int32_t sink, int32_t top_k,
                           float scale, int32_t select_splits, int32_t readers, int32_t* counters,
                           int64_t n_counters, void* scratch, size_t scratch_bytes, int32_t* lists,
                           int32_t* lengths, void* out, int32_t* status, void* stream);

/* lsa_decode_flat without caller buffers, for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart
 * in the reference. The counters and scratch live in a 16 MiB file-scope device array per
 * GPU (1 MiB of counters, 15 MiB of scratch); a call needing more returns
 * LSA_ERR_WORKSPACE. The library never allocates on this path. The first call on a device
 * clears the counters with a fill kernel on `stream`; every launch leaves them zero.
 * Calls share the device's array and keep its last contents: calls that overlap on one
 * GPU race and must not. reset_counters != 0 clears the whole 1 MiB counters region first
 * (after a launch that set *status: a late select workgroup of that launch may have left
 * keys anywhere its own shape reached). No slot map: the cache is not paged here. Arguments
 * and outputs otherwise as lsa_decode_flat. */
int lsa_decode_flat_noalloc(const void* q, const void* k, const void* v, int dtype, int64_t R, int64_t Tk,
                            int32_t Hq, int32_t Hkv, int32_t D, int64_t kv_batch_stride, int64_t kv_token_stride,
                            int64_t kv_head_stride, const void* centroids, const int32_t* members,
                            const int32_t* ends, int32_t table_flags, int32_t rows, int32_t cap, int64_t row_tables,
                            int64_t group_tables, int score_mode, const int32_t* positions,
                            int32_t cluster_block_size, int32_t block_buckets, int32_t top_p, int32_t window,
                            int32_t sink, int32_t top_k, float scale, int32_t select_splits, int32_t readers,
                            int32_t reset_counters, int32_t* lists, int32_t* lengths, void* out, int32_t* status,
                            void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LSA_ROCM_H */
