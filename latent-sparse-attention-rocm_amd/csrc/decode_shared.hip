// Entry points of the fused decode with one flat selection a row shared by every kv-head
// (reference pipeline.py:248-316 flat_select over the index space, then
// read_kernel_tiled.py:92-156; port/bench.py:147-153 `step`). The kernel is in
// decode_shared_impl.h.
#include "decode_shared_impl.h"

using namespace lsa;
using namespace lsa::shared;

extern "C" int64_t lsa_decode_shared_counters(int64_t R, int32_t Hkv, int32_t rows) {
  if (R <= 0 || Hkv <= 0 || rows <= 0 || rows > kShMaxRows) return 0;
  return sh_keys_at(R, Hkv) + 2 * R * (int64_t)rows;
}

extern "C" size_t lsa_decode_shared_scratch_bytes(int dtype, int64_t R, int32_t Hq, int32_t Hkv, int32_t D,
                                                  int32_t rows, int32_t top_p, int32_t window, int32_t sink,
                                                  int32_t top_k, int32_t readers) {
  if (rows <= 0 || top_p <= 0) return 0;
  return sh_scratch(dtype, R, Hq, Hkv, D, top_k, window, sink, readers);
}

extern "C" int lsa_decode_shared(const void* q, const void* k, const void* v, int dtype, int64_t R, int64_t Tk,
                                 int32_t Hq, int32_t Hkv, int32_t D, int64_t kv_batch_stride,
                                 int64_t kv_token_stride, int64_t kv_head_stride, const float* index_queries,
                                 const void* centroids, const int32_t* ends, int32_t table_flags, int32_t rows,
                                 int64_t row_tables, int score_mode, const int32_t* positions,
                                 const lsa_slot_map* slots, int32_t cluster_block_size, int32_t block_buckets,
                                 int32_t top_p, int32_t window, int32_t sink, int32_t top_k, float scale,
                                 int32_t select_splits, int32_t readers, int32_t* counters, int64_t n_counters,
                                 void* scratch, size_t scratch_bytes, int32_t* lists, int32_t* lengths, void* out,
                                 int32_t* status, void* stream) {
  const char* who = "lsa_decode_shared";
  SharedArgs a;
  LSA_TRY(sh_common(who, a, q, k, v, dtype, R, Tk, Hq, Hkv, D, kv_batch_stride, kv_token_stride, kv_head_stride,
                    index_queries, centroids, ends, table_flags, rows, row_tables, score_mode, positions, slots,
                    cluster_block_size, block_buckets, top_p, window, sink, top_k, scale, readers, counters, lists,
                    lengths, out, status));
  LSA_REQUIRE(rows <= kShMaxRows, LSA_ERR_SHAPE, "%s: tables of 1..%d buckets, got %d", who, kShMaxRows, rows);
  const int K = top_p < rows ? top_p : rows;
  LSA_REQUIRE(K <= kShMaxPicks, LSA_ERR_SHAPE, "%s: %d picks exceed %d", who, K, kShMaxPicks);
  a.K = K;
  a.kp = next_pow2(K);
  a.n_cols = rows;
  return sh_finish<false>(who, a, dtype, D, score_mode, select_splits, readers, sh_sel_bytes(rows, a.kp), counters,
                          n_counters, lsa_decode_shared_counters(R, Hkv, rows), scratch, scratch_bytes, stream);
}
