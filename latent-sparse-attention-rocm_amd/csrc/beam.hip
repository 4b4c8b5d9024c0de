// The multi-level beam select for gfx950 (reference _tree.py:318-373 _beam_pick_rows over
// the node levels of a hierarchy, with the per-row growth of _tree.py:100-142
// _growth_replay): one workgroup per (query row, group) walks the levels top-down.
//
// Growth (closed form of the replay for the row's page end = its visible bucket count V):
// the first covered = floor(V / node_block) * node_block buckets are under the made
// level-1 nodes [0, covered / node_size); a level's nodes close in whole blocks of
// node_block (closed = floor(made / node_block) * node_block) and make closed / node_size
// nodes of the level above, up to top_level levels, each capped by the nodes the table
// holds. The walk starts at the highest level with a made node, where every made node is
// a candidate; below it the candidates are the carried children of the kept nodes plus
// the level's open nodes [closed, made). Each candidate set is deduplicated (an LDS bitmap
// over ids), scored (the canonical score; on the matrix cores with an exact re-score when
// it fits screen_topk), the best beam_width kept (a tie to the lower id) and their
// children carried. At the buckets: the carried children below V plus the fresh buckets
// [covered, V), the best top_p, expanded in rank order like the flat select.
#include "lsa_abi_common.h"
#include "lsa_screen_dev.h"
#include "lsa_select_dev.h"

using namespace lsa;

namespace {

constexpr int kBeamSeenBits = 8192;       // ids a level (or the bucket table) may hold for the dedup bitmap
constexpr int kBeamMaxLdsKeys = 4096;     // candidates a level may score
constexpr size_t kBeamMaxDynLds = 40 * 1024;

struct BeamArgs {
  int64_t R;
  int G;
  const void* node_centroids[LSA_BEAM_MAX_LEVELS];  // level l + 1: [tables, n_nodes[l], D]
  const int32_t* children[LSA_BEAM_MAX_LEVELS];     // [tables, n_nodes[l], node_size]: rows of the level below
  int n_nodes[LSA_BEAM_MAX_LEVELS];
  int n_levels, node_size, node_block, beam;
  const void* centroids;
  const int32_t* members;
  const int32_t* ends;
  int rows, cap;
  int64_t row_tables, group_tables;
  const int32_t* positions;
  int cluster_block, block_buckets;
  int top_p, window, sink, top_k;
  int spans;   // bucket row j holds exactly ids ends[j - 1] .. ends[j] - 1 (ends[-1] = 0), top_p <= 64
  const int32_t* vends;  // the ends that decide visibility (nullptr: the closed-block rule)
  int screen;  // bf16 tables of a head dim screen_topk serves
  int cand_pow2, beam_pow2, top_pow2, carry_cap;
  SlotMap slots;  // a paged cache's slot table (table == nullptr: none)
  int32_t* lists;
  int32_t* lengths;
};

template <typename QT, typename CT, int SPAN>
__global__ __launch_bounds__(LSA_BLOCK) void select_beam_kernel(const QT* q, bool bf16_mode, BeamArgs a) {
  constexpr int D = 16 * SPAN;
  extern __shared__ uint64_t smem[];
  __shared__ RadixState st;
  __shared__ TopkScratch tks;
  __shared__ BinScratch bins;
  __shared__ ScreenLds scr;
  __shared__ uint32_t seen[kBeamSeenBits / 32];
  __shared__ int scan[LSA_WAVES];
  __shared__ int vis_lds[2 * LSA_WAVES];
  __shared__ int topk_ok;
  uint64_t* keys = smem;                                          // [cand_pow2]
  uint64_t* best = keys + a.cand_pow2;                            // [max(beam_pow2, top_pow2)]
  int32_t* cand = (int32_t*)(best + max(a.beam_pow2, a.top_pow2));  // [max(cand_pow2, top_p)]
  int32_t* carried = cand + max(a.cand_pow2, a.top_p);            // [carry_cap]
  const int64_t i = blockIdx.x;
  const int64_t r = (uint32_t)i / (uint32_t)a.G;
  const int g = (int)((uint32_t)i % (uint32_t)a.G);
  const int64_t position = a.positions[r];
  const int64_t t = r * a.row_tables + g * a.group_tables;
  float qs[SPAN];
  load_query_slice<QT, SPAN>(q + i * D, threadIdx.x & 15, bf16_mode, qs);
  const int visible =
      max(0, a.vends ? visible_count_block(position, a.rows, a.vends + t * a.rows, vis_lds)
                    : visible_count(position, a.rows, a.cluster_block, a.block_buckets, nullptr));

  // the row's growth
  int made[LSA_BEAM_MAX_LEVELS], closed[LSA_BEAM_MAX_LEVELS];
  int covered = visible / a.node_block * a.node_block;
  made[0] = covered / a.node_size;
  if (made[0] > a.n_nodes[0]) {
    made[0] = a.n_nodes[0];
    covered = made[0] * a.node_size;
  }
  int start = made[0] > 0 ? 1 : 0;
#pragma unroll
  for (int lv = 1; lv < LSA_BEAM_MAX_LEVELS; ++lv) {
    closed[lv - 1] = 0;
    made[lv] = 0;
    if (lv < a.n_levels) {
      closed[lv - 1] = made[lv - 1] / a.node_block * a.node_block;
      made[lv] = closed[lv - 1] / a.node_size;
      if (made[lv] > a.n_nodes[lv]) {
        made[lv] = a.n_nodes[lv];
        closed[lv - 1] = made[lv] * a.node_size;
      }
      if (made[lv] > 0) start = lv + 1;
    }
  }

  // the node levels, top-down
  int n_carried = 0;
  for (int lv = start; lv >= 1; --lv) {
    const int nn = a.n_nodes[lv - 1];
    const int first_open = lv == start ? 0 : closed[lv - 1];
    const int n_fresh = made[lv - 1] - first_open;
    const int n_cand = n_carried + n_fresh;  // <= cand_pow2 (host-checked)
    for (int x = threadIdx.x; x < (nn + 31) / 32; x += LSA_BLOCK) seen[x] = 0;
    __syncthreads();
    for (int j = threadIdx.x; j < a.cand_pow2; j += LSA_BLOCK) {  // each node once: the first lane to set its bit
      int32_t c = j < n_carried ? carried[j] : (j < n_cand ? first_open + (j - n_carried) : -1);
      if (c >= nn) c = -1;
      const uint32_t bit = 1u << (c & 31);
      cand[j] = (c >= 0 && !(atomicOr(&seen[c >> 5], bit) & bit)) ? c : -1;
    }
    __syncthreads();
    const CT* ncent = (const CT*)a.node_centroids[lv - 1] + t * (int64_t)nn * D;
    const int K = min(a.beam, a.cand_pow2);
    bool done = false;
    if constexpr (__is_same(CT, bf16_t) && SPAN >= 2 && SPAN <= 8) {
      if (a.screen && screen_pays(D, a.cand_pow2, K)) {
        screen_topk<D, 2>(
            qs, ncent, a.cand_pow2, [&](int j) { return cand[j]; }, [](int) { return true; }, K, a.beam_pow2, best,
            scr);
        done = true;
      }
    }
    if (!done) {
      score_keys<CT, SPAN>(qs, ncent, D, a.cand_pow2, [&](int j) { return cand[j]; }, keys);
      __syncthreads();
      block_topk_fast(keys, a.cand_pow2, K, a.beam_pow2, best, &tks, &st, &bins, &topk_ok);
    }
    // the kept nodes' children (rows of the level below) are carried
    const int32_t* kids = a.children[lv - 1] + t * (int64_t)nn * a.node_size;
    n_carried = K * a.node_size;  // <= carry_cap
    for (int j = threadIdx.x; j < n_carried; j += LSA_BLOCK) {
      const int node = key_column(u_to_key(best[j / a.node_size]));
      carried[j] = (node >= 0 && node < nn) ? kids[(int64_t)node * a.node_size + j % a.node_size] : -1;
    }
    __syncthreads();
  }

  // the buckets: carried children below the visible count, then the fresh buckets
  const int n_fresh = max(0, visible - covered);
  const int n_cand = n_carried + n_fresh;
  for (int x = threadIdx.x; x < (a.rows + 31) / 32; x += LSA_BLOCK) seen[x] = 0;
  __syncthreads();
  for (int j = threadIdx.x; j < a.cand_pow2; j += LSA_BLOCK) {
    int32_t c = j < n_carried ? carried[j] : (j < n_cand ? covered + (j - n_carried) : -1);
    if (c >= visible) c = -1;
    const uint32_t bit = 1u << (c & 31);
    cand[j] = (c >= 0 && !(atomicOr(&seen[c >> 5], bit) & bit)) ? c : -1;
  }
  __syncthreads();
  const CT* bcent = (const CT*)a.centroids + t * (int64_t)a.rows * D;
  const int K0 = min(a.top_p, a.cand_pow2);
  bool done0 = false;
  if constexpr (__is_same(CT, bf16_t) && SPAN >= 2 && SPAN <= 8) {
    if (a.screen && screen_pays(D, a.cand_pow2, K0)) {
      screen_topk<D, 2>(
          qs, bcent, a.cand_pow2, [&](int j) { return cand[j]; }, [](int) { return true; }, K0, a.top_pow2, best,
          scr);
      done0 = true;
    }
  }
  if (!done0) {
    score_keys<CT, SPAN>(qs, bcent, D, a.cand_pow2, [&](int j) { return cand[j]; }, keys);
    __syncthreads();
    block_topk_fast(keys, a.cand_pow2, K0, a.top_pow2, best, &tks, &st, &bins, &topk_ok);
  }
  for (int j = threadIdx.x; j < a.top_p; j += LSA_BLOCK) cand[j] = j < K0 ? key_column(u_to_key(best[j])) : -1;
  __syncthreads();
  const int width = a.top_k + a.window + a.sink;
  const SlotRow map = slot_row_of(a.slots, r);
  int len;
  if (a.spans && a.top_p <= LSA_WAVE) {  // span tables: kept ids from the picks' span ends, no member rows
    __shared__ int span_lds[2 * LSA_WAVE + 1];
    len = expand_spans(cand, a.top_p, a.ends + t * a.rows, a.rows, position, a.window, a.sink, a.top_k,
                       a.lists + i * width, width, span_lds, map);
  } else if (a.spans) {
    len = a.top_p <= 4 * LSA_BLOCK
              ? expand_spans_wide<4>(cand, a.top_p, a.ends + t * a.rows, a.rows, position, a.window, a.sink,
                                     a.top_k, a.lists + i * width, width, nullptr, scan, map)
              : expand_spans_wide<16>(cand, a.top_p, a.ends + t * a.rows, a.rows, position, a.window, a.sink,
                                      a.top_k, a.lists + i * width, width, nullptr, scan, map);
  } else {
    const int32_t* tab = a.members + t * (int64_t)a.rows * a.cap;
    len = expand_walk(cand, a.top_p, tab, a.rows, a.cap, position, a.window, a.sink, a.top_k, a.lists + i * width,
                      width, scan, nullptr, map);
  }
  if (threadIdx.x == 0) a.lengths[i] = len;
}

}  // namespace

extern "C" int lsa_select_beam(const void* queries, int q_dtype, int64_t R, int32_t G, int32_t D, int32_t n_levels,
                               const void* const* node_centroids, const int32_t* const* children,
                               const int32_t* n_nodes, int32_t node_size, int32_t node_block, int32_t top_level,
                               const void* centroids, const int32_t* members, const int32_t* ends,
                               int32_t table_flags, int32_t rows, int32_t cap, int64_t row_tables,
                               int64_t group_tables, int score_mode, const int32_t* positions,
                               const lsa_slot_map* slots, int32_t cluster_block_size, int32_t block_buckets,
                               int32_t beam_width, int32_t top_p, int32_t window, int32_t sink, int32_t top_k,
                               int32_t* lists, int32_t* lengths, void* stream) {
  LSA_REQUIRE(queries && node_centroids && children && n_nodes && centroids && members && positions && lists &&
                  lengths,
              LSA_ERR_NULL, "lsa_select_beam: NULL pointer");
  SlotMap sm;
  LSA_TRY(check_slots("lsa_select_beam", slots, &sm));
  LSA_TRY(check_dtype(q_dtype));
  LSA_TRY(check_dim(D));
  LSA_TRY(check_tables(rows, cap, row_tables, group_tables));
  LSA_REQUIRE(score_mode == LSA_SCORE_BF16 || score_mode == LSA_SCORE_F32, LSA_ERR_DTYPE, "bad score mode");
  LSA_TRY(check_aligned(centroids, D, score_mode, members, cap));
  LSA_TRY(check_query_aligned(queries, q_dtype, D));
  LSA_REQUIRE(R >= 0 && G >= 1 && R * G <= 0x7FFFFFFF, LSA_ERR_SHAPE, "lsa_select_beam: bad sizes");
  LSA_REQUIRE(n_levels >= 1 && n_levels <= LSA_BEAM_MAX_LEVELS, LSA_ERR_SHAPE,
              "lsa_select_beam: 1 to %d node levels, got %d", LSA_BEAM_MAX_LEVELS, n_levels);
  LSA_REQUIRE(top_level >= 1, LSA_ERR_SHAPE, "lsa_select_beam: top_level must be >= 1, got %d", top_level);
  LSA_REQUIRE(node_size >= 1 && node_block >= node_size && node_block % node_size == 0, LSA_ERR_SHAPE,
              "lsa_select_beam: node_block (%d) must be a positive multiple of node_size (%d)", node_block,
              node_size);
  LSA_REQUIRE(rows <= kBeamSeenBits, LSA_ERR_SHAPE, "lsa_select_beam: %d buckets a table exceed %d", rows,
              kBeamSeenBits);
  LSA_REQUIRE(beam_width >= 1 && top_p >= 1 && window >= 0 && sink >= 0 && top_k >= 0, LSA_ERR_SHAPE,
              "lsa_select_beam: beam_width, top_p >= 1; window, sink, top_k >= 0");
  LSA_REQUIRE(ends || cluster_block_size >= 1, LSA_ERR_SHAPE, "lsa_select_beam: cluster_block_size must be >= 1");
  LSA_REQUIRE((table_flags & ~(LSA_TABLE_SPANS | LSA_TABLE_BLOCK_VISIBLE)) == 0, LSA_ERR_SHAPE,
              "lsa_select_beam: unknown table flags %d", table_flags);
  LSA_REQUIRE(!(table_flags & LSA_TABLE_BLOCK_VISIBLE) || cluster_block_size >= 1, LSA_ERR_SHAPE,
              "lsa_select_beam: cluster_block_size must be >= 1");
  LSA_REQUIRE(!(table_flags & LSA_TABLE_SPANS) || ends, LSA_ERR_SHAPE,
              "lsa_select_beam: LSA_TABLE_SPANS needs the span ends");
  const int levels = n_levels < top_level ? n_levels : top_level;
  for (int l = 0; l < levels; ++l) {
    LSA_REQUIRE(node_centroids[l] && children[l], LSA_ERR_NULL, "lsa_select_beam: level %d: NULL pointer", l + 1);
    LSA_REQUIRE(n_nodes[l] >= 1 && n_nodes[l] <= kBeamSeenBits, LSA_ERR_SHAPE,
                "lsa_select_beam: level %d holds %d nodes (1 to %d)", l + 1, n_nodes[l], kBeamSeenBits);
    LSA_TRY(check_aligned(node_centroids[l], D, score_mode, nullptr, cap));
  }
  // The most candidates a level scores: at the start level its made nodes (every node of
  // the top level; below the top, fewer than node_block, or the level above would hold a
  // made node); below the start, the carried children plus the open nodes [closed, made)
  // (fewer than node_block unless the level above is full); at the buckets the carried
  // children plus the fresh buckets [covered, V).
  const int64_t carry = (int64_t)beam_width * node_size;
  int64_t most = n_nodes[levels - 1] > node_block - 1 ? n_nodes[levels - 1] : node_block - 1;
  for (int l = 0; l < levels; ++l) {
    const int64_t below = l == 0 ? rows : n_nodes[l - 1];
    const int64_t past = below - (int64_t)n_nodes[l] * node_size;
    int64_t open = past > node_block - 1 ? past : node_block - 1;
    open = open < below ? open : below;
    most = carry + open > most ? carry + open : most;
  }
  LSA_REQUIRE(most <= kBeamMaxLdsKeys, LSA_ERR_SHAPE, "lsa_select_beam: %lld candidates a level exceed %d",
              (long long)most, kBeamMaxLdsKeys);
  if (R * G == 0) return LSA_OK;
  BeamArgs a;
  a.R = R; a.G = G;
  for (int l = 0; l < LSA_BEAM_MAX_LEVELS; ++l) {
    a.node_centroids[l] = l < levels ? node_centroids[l] : nullptr;
    a.children[l] = l < levels ? children[l] : nullptr;
    a.n_nodes[l] = l < levels ? n_nodes[l] : 0;
  }
  a.n_levels = levels; a.node_size = node_size; a.node_block = node_block; a.beam = beam_width;
  a.centroids = centroids; a.members = members; a.ends = ends; a.rows = rows; a.cap = cap;
  a.vends = (table_flags & LSA_TABLE_BLOCK_VISIBLE) ? nullptr : ends;
  a.row_tables = row_tables; a.group_tables = group_tables; a.positions = positions;
  a.cluster_block = cluster_block_size; a.block_buckets = block_buckets;
  a.top_p = top_p; a.window = window; a.sink = sink; a.top_k = top_k;
  a.spans = (table_flags & LSA_TABLE_SPANS) && top_p <= 16 * LSA_BLOCK ? 1 : 0;  // else the member rows
  a.screen = score_mode == LSA_SCORE_BF16 && (D == 32 || D == 64 || D == 128) ? 1 : 0;
  a.cand_pow2 = next_pow2((int)most);
  a.beam_pow2 = next_pow2(beam_width < a.cand_pow2 ? beam_width : a.cand_pow2);
  a.top_pow2 = next_pow2(top_p < a.cand_pow2 ? top_p : a.cand_pow2);
  a.carry_cap = (beam_width < a.cand_pow2 ? beam_width : a.cand_pow2) * node_size;
  a.lists = lists; a.lengths = lengths; a.slots = sm;
  const int best_slots = a.beam_pow2 > a.top_pow2 ? a.beam_pow2 : a.top_pow2;
  const int cand_slots = a.cand_pow2 > top_p ? a.cand_pow2 : top_p;
  const size_t shmem = sizeof(uint64_t) * (size_t)(a.cand_pow2 + best_slots) +
                       sizeof(int32_t) * (size_t)(cand_slots + a.carry_cap);
  LSA_REQUIRE(shmem <= kBeamMaxDynLds, LSA_ERR_SHAPE, "lsa_select_beam: %zu bytes of LDS needed (at most %zu)", shmem,
              kBeamMaxDynLds);
  const bool bf16 = score_mode == LSA_SCORE_BF16;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)(R * G));
  LSA_DISPATCH_QT(q_dtype, LSA_DISPATCH_SPAN(D / 16, {
    if (bf16) select_beam_kernel<QT, bf16_t, SPAN><<<grid, LSA_BLOCK, shmem, s>>>((const QT*)queries, true, a);
    else select_beam_kernel<QT, float, SPAN><<<grid, LSA_BLOCK, shmem, s>>>((const QT*)queries, false, a);
  }))
  LSA_LAUNCHED("lsa_select_beam");
  return LSA_OK;
}
