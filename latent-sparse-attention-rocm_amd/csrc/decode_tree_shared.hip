// Entry points of the fused decode with one multi-level beam selection a row shared by
// every kv-head (reference pipeline.py:319-337 tree_select over the index space, then
// read_kernel_tiled.py:92-156; port/bench.py:147-153 `step` with the tree arm). The kernel
// is in decode_shared_impl.h.
#include "decode_shared_impl.h"

using namespace lsa;
using namespace lsa::shared;

extern "C" int64_t lsa_decode_tree_shared_counters(int64_t R, int32_t Hkv, int32_t n_levels, const int32_t* n_nodes,
                                                   int32_t rows) {
  if (R <= 0 || Hkv <= 0 || rows <= 0 || n_levels < 1 || n_levels > LSA_BEAM_MAX_LEVELS || !n_nodes) return 0;
  int64_t cols = rows;
  for (int l = 0; l < n_levels; ++l) {
    if (n_nodes[l] < 1) return 0;
    cols += n_nodes[l];
  }
  return sh_keys_at(R, Hkv) + 2 * R * cols;
}

extern "C" int lsa_decode_tree_shared(const void* q, const void* k, const void* v, int dtype, int64_t R, int64_t Tk,
                                      int32_t Hq, int32_t Hkv, int32_t D, int64_t kv_batch_stride,
                                      int64_t kv_token_stride, int64_t kv_head_stride, const float* index_queries,
                                      int32_t n_levels, const void* const* node_centroids,
                                      const int32_t* const* children, const int32_t* n_nodes, int32_t node_size,
                                      int32_t node_block, int32_t top_level, const void* centroids,
                                      const int32_t* ends, int32_t table_flags, int32_t rows, int64_t row_tables,
                                      int score_mode, const int32_t* positions, const lsa_slot_map* slots,
                                      int32_t cluster_block_size, int32_t block_buckets, int32_t beam_width,
                                      int32_t top_p, int32_t window, int32_t sink, int32_t top_k, float scale,
                                      int32_t select_splits, int32_t readers, int32_t* counters, int64_t n_counters,
                                      void* scratch, size_t scratch_bytes, int32_t* lists, int32_t* lengths,
                                      void* out, int32_t* status, void* stream) {
  const char* who = "lsa_decode_tree_shared";
  SharedArgs a;
  LSA_TRY(sh_common(who, a, q, k, v, dtype, R, Tk, Hq, Hkv, D, kv_batch_stride, kv_token_stride, kv_head_stride,
                    index_queries, centroids, ends, table_flags, rows, row_tables, score_mode, positions, slots,
                    cluster_block_size, block_buckets, top_p, window, sink, top_k, scale, readers, counters, lists,
                    lengths, out, status));
  LSA_REQUIRE(node_centroids && children && n_nodes, LSA_ERR_NULL, "%s: NULL pointer", who);
  LSA_REQUIRE(n_levels >= 1 && n_levels <= LSA_BEAM_MAX_LEVELS, LSA_ERR_SHAPE, "%s: 1 to %d node levels, got %d",
              who, LSA_BEAM_MAX_LEVELS, n_levels);
  LSA_REQUIRE(top_level >= 1, LSA_ERR_SHAPE, "%s: top_level must be >= 1, got %d", who, top_level);
  LSA_REQUIRE(node_size >= 1 && node_block >= node_size && node_block % node_size == 0, LSA_ERR_SHAPE,
              "%s: node_block (%d) must be a positive multiple of node_size (%d)", who, node_block, node_size);
  LSA_REQUIRE(rows <= kShSeenBits, LSA_ERR_SHAPE, "%s: %d buckets a table exceed %d", who, rows, kShSeenBits);
  LSA_REQUIRE(beam_width >= 1, LSA_ERR_SHAPE, "%s: beam_width >= 1", who);
  const int levels = n_levels < top_level ? n_levels : top_level;
  const size_t esize = score_mode == LSA_SCORE_F32 ? 4 : 2;
  const size_t align = esize * D / 16 > 16 ? 16 : esize * D / 16;
  int64_t cols = 0;
  for (int l = 0; l < levels; ++l) {
    LSA_REQUIRE(node_centroids[l] && children[l], LSA_ERR_NULL, "%s: level %d: NULL pointer", who, l + 1);
    LSA_REQUIRE(n_nodes[l] >= 1 && n_nodes[l] <= kShSeenBits, LSA_ERR_SHAPE, "%s: level %d holds %d nodes (1 to %d)",
                who, l + 1, n_nodes[l], kShSeenBits);
    LSA_REQUIRE(((uintptr_t)node_centroids[l] % align) == 0, LSA_ERR_ALIGN,
                "%s: level %d centroid table must be %zu-byte aligned", who, l + 1, align);
    a.node_centroids[l] = node_centroids[l];
    a.children[l] = children[l];
    a.n_nodes[l] = n_nodes[l];
    a.col_base[l] = cols;
    cols += n_nodes[l];
  }
  a.col_base[levels] = cols;
  a.n_cols = cols + rows;
  const int64_t most = tree_most(levels, n_nodes, rows, node_size, node_block, beam_width);
  LSA_REQUIRE(most <= kShMaxCand, LSA_ERR_SHAPE, "%s: %lld candidates a level exceed %d", who, (long long)most,
              kShMaxCand);
  a.n_levels = levels; a.node_size = node_size; a.node_block = node_block; a.beam = beam_width;
  a.cand_pow2 = next_pow2((int)most);
  a.beam_pow2 = next_pow2(beam_width < a.cand_pow2 ? beam_width : a.cand_pow2);
  a.carry_cap = (beam_width < a.cand_pow2 ? beam_width : a.cand_pow2) * node_size;
  a.K = top_p < a.cand_pow2 ? top_p : a.cand_pow2;
  LSA_REQUIRE(a.K <= kShMaxPicks, LSA_ERR_SHAPE, "%s: %d picks exceed %d", who, a.K, kShMaxPicks);
  a.kp = next_pow2(a.K);
  // the walk reads the published keys from LDS when their score halves fit beside it
  const int best_slots = a.kp > a.beam_pow2 ? a.kp : a.beam_pow2;
  const int span = lsa_read_tile_tokens(dtype, D, Hq / Hkv);
  const size_t cached = sh_region_at(a.kp) + tree_lds(a.cand_pow2, best_slots, a.carry_cap, a.n_cols).end;
  a.cache_keys = span > 0 && cached <= kShMaxLds ? 1 : 0;
  const TreeLds L = tree_lds(a.cand_pow2, best_slots, a.carry_cap, a.cache_keys ? a.n_cols : 0);
  return sh_finish<true>(who, a, dtype, D, score_mode, select_splits, readers, L.end, counters, n_counters,
                         lsa_decode_tree_shared_counters(R, Hkv, levels, n_nodes, rows), scratch, scratch_bytes,
                         stream);
}
