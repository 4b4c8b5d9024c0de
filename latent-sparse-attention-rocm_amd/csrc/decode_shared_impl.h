// Fused decode step with one selection a query row shared by every kv-head, for gfx950
// (the kernel and its host checks; decode_shared.hip and decode_tree_shared.hip hold the
// flat and the tree entry points):
// the reference's own layout (one index-space table and one index query a position, the
// lists shared by every head: pipeline.py:248-316 flat_select or pipeline.py:319-337
// tree_select over the index space, then read_kernel_tiled.py:92-156 with [B, Tq, W]
// lists; port/bench.py:147-153 `step`) at its own knobs (PortConfig, pipeline.py:32-54: up
// to 4096 buckets, top_p 1024, top_k 4096; the tree's 3 node levels and beam 64).
//
// The 1-D grid holds S select workgroups a row, then NR readers for every (row, kv-head)
// unit (unit fastest).
//
// Select workgroup (row r, split s): scores its columns with the row's fp32 index query
// (the canonical score) and publishes each column's key + 1 (nonzero once written) with
// device-scope stores. It never waits. Flat: columns of the bucket table, visibility (span
// ends or closed blocks) applied (an invisible bucket publishes EMPTY). Tree: the columns
// of every node level and then of the bucket table, with no visibility: the walk below
// decides which of them it reads.
//
// Reader (unit (r, g), role): loads its kv-head's query rows and (a paged cache) warms the
// slot-table row in its XCD's L2, then selects:
//  - flat: the table's span ends go to LDS; every wave polls its share of the row's keys
//    (16 a lane, all in flight each round) until all are written; the keys stay in
//    registers and the block ranks them (topk_bins_regs; a register radix select when a
//    score is not finite or a bin is crowded);
//  - tree: the multi-level beam walk (the row's growth from its visible bucket count; at
//    each level the candidates deduplicated through an LDS bitmap, their keys gathered
//    from the published ones, the best beam kept and their children carried; at the
//    buckets the carried children below the visible count plus the fresh buckets, the best
//    top_p).
// Waits are bounded: past the spin limit a reader sets *status, arrives and exits. Then
// each pick's kept range [max(begin, sink), min(end, window start)) from the span ends,
// placed by one block scan (clipped at top_k); the reader reads its contiguous run of the
// list's tiles: ids expanded (and mapped through the slot table), written to the shared
// list by kv-head 0's readers, gathered with the pipelined tile loop. Partials are combined
// by the unit's last reader; the last unit of a row to finish clears the row's published
// keys, so every launch finds them zero.
//
// Readers wait only on select workgroups, which hold lower ids and never wait: dispatched
// in id order, the select workgroups are resident (or done) before any reader holds a slot.
#pragma once
#include "lsa_abi_common.h"
#include "decode_dev.h"

namespace lsa {
namespace shared {

using namespace lsa::decode;

constexpr int kShMaxRows = 16 * LSA_BLOCK;  // flat: buckets a table (16 keys a reader thread holds)
constexpr int kShMaxPicks = 4 * LSA_BLOCK;  // picks: 4 a thread in the placement scan
constexpr int kShMaxReaders = 64;           // readers a unit (split partials of the combine)
constexpr size_t kShMaxLds = 64 * 1024;
constexpr int kShSeenBits = 8192;           // tree: ids a level (or the bucket table) may hold
constexpr int kShMaxCand = 16 * LSA_BLOCK;  // tree: candidates a level may score (16 a thread)

struct SharedArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  int64_t R;
  int G, Hq;
  int64_t Tk, kv_sb, kv_st, kv_sh;
  const float* idx_q;       // [R, D] fp32 index queries
  const void* centroids;    // [tables, rows, D], the scoring type
  const int32_t* ends;      // [tables, rows] span ends
  const int32_t* vends;     // the ends that decide visibility (nullptr: the closed-block rule)
  int rows;
  int64_t row_tables;       // table of row r: r * row_tables
  const int32_t* positions;
  int cluster_block, block_buckets;
  int K, kp;                // picks (flat: min(top_p, rows); tree: min(top_p, cand_pow2)), their slots
  int window, sink, top_k, W;
  int S, cs;                // select workgroups a row, columns each
  int span, NR;             // slots a read tile, readers a unit
  float scale_log2;
  int spin_limit;
  int skip_publish;         // test hook: the select workgroups never publish (readers give up)
  int64_t n_cols;           // keys published a row
  uint64_t* pub;            // [R][n_cols] published keys + 1 (0: not yet written)
  int* rd_count;            // [R * G] reader arrivals
  int* done;                // [R] units of a row finished
  float* ws_part;           // [R * G][NR][GQ * (D + 2)]
  int32_t* lists;           // [R][W]
  int32_t* lengths;         // [R]
  int32_t* status;
  SlotMap slots;
  // tree: node level l + 1 (l = 0 .. n_levels - 1, bottom up): centroids [tables,
  // n_nodes[l], D], children [tables, n_nodes[l], node_size] (rows of the level below;
  // bucket rows for l = 0)
  int n_levels;
  const void* node_centroids[LSA_BEAM_MAX_LEVELS];
  const int32_t* children[LSA_BEAM_MAX_LEVELS];
  int n_nodes[LSA_BEAM_MAX_LEVELS];
  int64_t col_base[LSA_BEAM_MAX_LEVELS + 1];  // first published column of each level, then of the buckets
  int node_size, node_block, beam;
  int cand_pow2, beam_pow2, carry_cap;
  int cache_keys;           // the published keys' score halves are copied to LDS once
};

// Reader LDS: a header, the picks (first kept id and first list slot of each), then a
// region the selection phase and the read phase (ids of a chunk, the read's merge state)
// take in turn.
struct ShHdr {
  int filled, last, ok;
  int wbad[LSA_WAVES];
  int scan[LSA_WAVES];
  int vis[2 * LSA_WAVES];
};
constexpr size_t a16(size_t x) { return (x + 15) & ~(size_t)15; }
__host__ __device__ inline size_t sh_picks_at() { return a16(sizeof(ShHdr)); }
__host__ __device__ inline size_t sh_region_at(int kp) { return sh_picks_at() + a16(sizeof(int32_t) * (2 * (size_t)kp + 1)); }
// top-K state: the flat reader bins its thousands of keys finer (BinScratchWide)
__host__ __device__ inline size_t sh_scratch_bytes(bool wide) {
  return a16(sizeof(TopkScratch)) + a16(wide ? sizeof(BinScratchWide) : sizeof(BinScratch)) + a16(sizeof(RadixState));
}
// flat selection phase, within the region: span ends, sorted keys, candidates, top-K state
__host__ __device__ inline size_t sh_best_at(int rows) { return a16(sizeof(int32_t) * (size_t)rows); }
__host__ __device__ inline size_t sh_cand_at(int rows, int kp) { return sh_best_at(rows) + sizeof(uint64_t) * (size_t)kp; }
__host__ __device__ inline size_t sh_topk_at(int rows, int kp) {
  return a16(sh_cand_at(rows, kp) + sizeof(uint64_t) * ((size_t)kp + LSA_WAVE));
}
__host__ __device__ inline size_t sh_sel_bytes(int rows, int kp) { return sh_topk_at(rows, kp) + sh_scratch_bytes(true); }
// tree selection phase, within the region: a level's keys, the sorted keys, candidates,
// carried children, the dedup bitmap, top-K state, then (cache_cols > 0) the high halves
// of the row's published keys
struct TreeLds {
  size_t keys, best, cand, carried, seen, topk, cache, end;
};
__host__ __device__ inline TreeLds tree_lds(int cand_pow2, int best_slots, int carry_cap, int64_t cache_cols) {
  TreeLds L;
  L.keys = 0;
  L.best = L.keys + sizeof(uint64_t) * (size_t)cand_pow2;
  L.cand = L.best + sizeof(uint64_t) * (size_t)best_slots;
  L.carried = a16(L.cand + sizeof(int32_t) * (size_t)cand_pow2);
  L.seen = a16(L.carried + sizeof(int32_t) * (size_t)carry_cap);
  L.topk = a16(L.seen + sizeof(uint32_t) * (size_t)(kShSeenBits / 32));
  L.cache = a16(L.topk + sh_scratch_bytes(false));
  L.end = L.cache + sizeof(uint32_t) * (size_t)cache_cols;
  return L;
}
// read phase, within the region: ids of a chunk, then the merge state
constexpr int kShChunkTiles = 32;
__host__ __device__ inline size_t sh_rd_at(int span) { return a16(sizeof(int32_t) * (size_t)kShChunkTiles * span); }
template <int D, int GQ>
__host__ __device__ inline size_t sh_read_bytes(int span) {
  return sh_rd_at(span) + sizeof(ReadLds<D, GQ, kShMaxReaders>);
}

template <typename CT, int D, bool TREE>
__device__ __forceinline__ void shared_select(const SharedArgs& a, char* smem, int64_t r, int s) {
  constexpr int SPAN = D / 16;
  uint64_t* keys = (uint64_t*)smem;  // [cs]
  const int tid = threadIdx.x;
  const int64_t position = a.positions[r];
  const int64_t t = r * a.row_tables;
  const int64_t c0 = (int64_t)s * a.cs;
  const int64_t c1 = c0 + a.cs < a.n_cols ? c0 + a.cs : a.n_cols;
  const int n_local = c1 > c0 ? (int)(c1 - c0) : 0;
  float qs[SPAN];
  load_query_slice<float, SPAN>(a.idx_q + r * D, tid & 15, __is_same(CT, bf16_t), qs);
  if constexpr (!TREE) {
    const CT* cent = (const CT*)a.centroids + t * a.rows * (int64_t)D;
    const int32_t* vends = a.vends ? a.vends + t * a.rows : nullptr;
    const int vis = vends ? 0 : visible_closed(position, a.rows, a.cluster_block, a.block_buckets);
    const int64_t lim = position + 1;
    const int b0 = (int)c0;
    score_keys<CT, SPAN>(
        qs, cent, D, n_local, [&](int j) { return b0 + j; },
        [&](int j) { return vends ? (int64_t)vends[b0 + j] <= lim : b0 + j < vis; }, keys);
  } else {
    // the node levels' columns, then the buckets': one score_keys pass a table the slice meets
    for (int seg = 0; seg <= a.n_levels; ++seg) {
      const int64_t s0 = a.col_base[seg], s1 = seg < a.n_levels ? a.col_base[seg + 1] : a.n_cols;
      const int64_t lo = c0 > s0 ? c0 : s0, hi = c1 < s1 ? c1 : s1;
      if (lo >= hi) continue;
      const int n_tab = seg < a.n_levels ? a.n_nodes[seg] : a.rows;
      const CT* cent = (const CT*)(seg < a.n_levels ? a.node_centroids[seg] : a.centroids) + t * n_tab * (int64_t)D;
      const int first = (int)(lo - s0);
      score_keys<CT, SPAN>(qs, cent, D, (int)(hi - lo), [&](int j) { return first + j; }, keys + (lo - c0));
    }
  }
  __syncthreads();
  DECODE_MARK(1);
  if (a.skip_publish) return;
  uint64_t* mine = a.pub + r * a.n_cols + c0;
  for (int j = tid; j < n_local; j += LSA_BLOCK) coherent_store_u64(mine + j, keys[j] + 1);
  DECODE_MARK(6);
}

// The unit's last reader: the row's keys are cleared once every kv-head's unit is done.
__device__ __forceinline__ void shared_unit_done(const SharedArgs& a, ShHdr& hd, int64_t r) {
  if (threadIdx.x == 0) {
    const int before = __hip_atomic_fetch_add(&a.done[r], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    hd.last = before == a.G - 1;
    if (hd.last) __hip_atomic_store(&a.done[r], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (hd.last) {
    uint64_t* pub = a.pub + r * a.n_cols;
    for (int64_t x = threadIdx.x; x < a.n_cols; x += LSA_BLOCK) coherent_store_u64(pub + x, 0);
  }
}

// Every wave's verdict on a bounded wait, shared: true (every thread) when one gave up.
__device__ __forceinline__ bool block_gave_up(ShHdr& hd, int bad) {
  if ((threadIdx.x & (LSA_WAVE - 1)) == 0) hd.wbad[threadIdx.x / LSA_WAVE] = bad;
  __syncthreads();
  return (hd.wbad[0] | hd.wbad[1] | hd.wbad[2] | hd.wbad[3]) != 0;
}

// One tree level's candidate list: the carried entries [0, n_carried), then the ids
// first .. first + (n_cand - n_carried) - 1; ids outside [0, limit) and repeats (the first
// entry to claim an id keeps it) become -1. n_ids: the ids the bitmap must clear.
__device__ __forceinline__ void tree_candidates(int32_t* cand, uint32_t* seen, int n_ids, int limit,
                                                const int32_t* carried, int n_carried, int first, int n_cand,
                                                int cand_pow2) {
  for (int x = threadIdx.x; x < (n_ids + 31) / 32; x += LSA_BLOCK) seen[x] = 0;
  __syncthreads();
  for (int j = threadIdx.x; j < cand_pow2; j += LSA_BLOCK) {
    int32_t c = j < n_carried ? carried[j] : (j < n_cand ? first + (j - n_carried) : -1);
    if (c >= limit) c = -1;
    const uint32_t bit = 1u << (c & 31);
    cand[j] = (c >= 0 && !(atomicOr(&seen[c >> 5], bit) & bit)) ? c : -1;
  }
  __syncthreads();
}

// Keys of a level's candidates cand[0..n) from the published ones (EMPTY for -1 entries),
// every load of a round in flight together, polled until written; false (every thread)
// when a wave gave up at the spin limit.
__device__ __forceinline__ bool tree_gather(const SharedArgs& a, ShHdr& hd, const uint64_t* pub,
                                            const int32_t* cand, int n, uint64_t* keys) {
  constexpr int GPT = kShMaxCand / LSA_BLOCK;
  const int tid = threadIdx.x;
  int32_t c[GPT];
  uint64_t x[GPT];
#pragma unroll
  for (int m = 0; m < GPT; ++m) {
    const int j = m * LSA_BLOCK + tid;
    c[m] = j < n ? cand[j] : -1;
    x[m] = 0;
  }
  int bad = 0;
  for (int it = 0;; ++it) {
    bool ok = true;
#pragma unroll
    for (int m = 0; m < GPT; ++m) {
      if (m * LSA_BLOCK < n) {  // uniform
        x[m] = coherent_load_u64(pub + (c[m] >= 0 ? c[m] : 0));
        ok &= c[m] < 0 || x[m] != 0;
      }
    }
    if (__all(ok)) break;
    if (it >= a.spin_limit) {
      bad = 1;
      break;
    }
    __builtin_amdgcn_s_sleep(2);
  }
#pragma unroll
  for (int m = 0; m < GPT; ++m) {
    const int j = m * LSA_BLOCK + tid;
    if (j < n) keys[j] = c[m] >= 0 ? x[m] - 1 : 0;
  }
  return !block_gave_up(hd, bad);
}

// The row's published keys, polled until written (every load of a round in flight
// together, 24 a thread a round), their high halves (the ordered score bits) kept in
// cache[0..n_cols): a key is rebuilt from its column. False (every thread) when a wave gave
// up at the spin limit.
__device__ __forceinline__ bool tree_cache(const SharedArgs& a, ShHdr& hd, const uint64_t* pub, uint32_t* cache) {
  constexpr int CPT = 24;
  const int tid = threadIdx.x;
  int bad = 0;
  for (int64_t base = 0; base < a.n_cols && !bad; base += CPT * LSA_BLOCK) {
    uint64_t x[CPT];
    for (int it = 0;; ++it) {
      bool ok = true;
#pragma unroll
      for (int m = 0; m < CPT; ++m) {
        const int64_t j = base + m * LSA_BLOCK + tid;
        x[m] = coherent_load_u64(pub + (j < a.n_cols ? j : 0));
        ok &= j >= a.n_cols || x[m] != 0;
      }
      if (__all(ok)) break;
      if (it >= a.spin_limit) {
        bad = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
#pragma unroll
    for (int m = 0; m < CPT; ++m) {
      const int64_t j = base + m * LSA_BLOCK + tid;
      if (j < a.n_cols) cache[j] = (uint32_t)((x[m] - 1) >> 32);
    }
  }
  return !block_gave_up(hd, bad);
}

// Keys of a level's candidates cand[0..n) rebuilt from the cached score halves of its
// columns (EMPTY for -1 entries): u = (score half << 32) | (0x7FFFFFFF - column).
__device__ __forceinline__ void tree_gather_cached(const uint32_t* cache, const int32_t* cand, int n,
                                                   uint64_t* keys) {
  for (int j = threadIdx.x; j < n; j += LSA_BLOCK) {
    const int32_t c = cand[j];
    keys[j] = c >= 0 ? ((uint64_t)cache[c] << 32) | (uint64_t)(uint32_t)(0x7FFFFFFF - c) : 0;
  }
  __syncthreads();
}

// The multi-level beam walk of row r (reference _tree.py:318-373 _beam_pick_rows with the
// growth of _tree.py:100-142 at page end V = the visible bucket count): best[0..kp) gets
// the picked buckets' keys, sorted. False when a wait gave up.
__device__ __forceinline__ bool tree_walk(const SharedArgs& a, ShHdr& hd, char* region, int64_t r, int64_t t,
                                          int64_t position, uint64_t* best) {
  const TreeLds L =
      tree_lds(a.cand_pow2, a.kp > a.beam_pow2 ? a.kp : a.beam_pow2, a.carry_cap, a.cache_keys ? a.n_cols : 0);
  uint64_t* keys = (uint64_t*)(region + L.keys);
  uint32_t* cache = (uint32_t*)(region + L.cache);
  int32_t* cand = (int32_t*)(region + L.cand);
  int32_t* carried = (int32_t*)(region + L.carried);
  uint32_t* seen = (uint32_t*)(region + L.seen);
  TopkScratch* tks = (TopkScratch*)(region + L.topk);
  BinScratch* bins = (BinScratch*)((char*)tks + a16(sizeof(TopkScratch)));
  RadixState* rst = (RadixState*)((char*)bins + a16(sizeof(BinScratch)));
  const int visible =
      max(0, a.vends ? visible_count_block(position, a.rows, a.vends + t * a.rows, hd.vis)
                     : visible_count(position, a.rows, a.cluster_block, a.block_buckets, nullptr));

  // the row's growth: covered buckets make level-1 nodes; a level's nodes close in whole
  // node blocks and make nodes of the level above, each level capped by its table
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

  const uint64_t* pub = a.pub + r * a.n_cols;
  if (a.cache_keys && !tree_cache(a, hd, pub, cache)) return false;
  const int ns = a.node_size;
  int n_carried = 0;
  for (int lv = start; lv >= 1; --lv) {  // the node levels, top-down
    const int nn = a.n_nodes[lv - 1];
    const int first_open = lv == start ? 0 : closed[lv - 1];
    tree_candidates(cand, seen, nn, nn, carried, n_carried, first_open, n_carried + made[lv - 1] - first_open,
                    a.cand_pow2);
    if (a.cache_keys) tree_gather_cached(cache + a.col_base[lv - 1], cand, a.cand_pow2, keys);
    else if (!tree_gather(a, hd, pub + a.col_base[lv - 1], cand, a.cand_pow2, keys)) return false;
    const int K = a.beam < a.cand_pow2 ? a.beam : a.cand_pow2;
    block_topk_fast(keys, a.cand_pow2, K, a.beam_pow2, best, tks, rst, bins, &hd.ok);
    const int32_t* kids = a.children[lv - 1] + t * (int64_t)nn * ns;
    n_carried = K * ns;  // <= carry_cap
    for (int j = threadIdx.x; j < n_carried; j += LSA_BLOCK) {
      const int node = key_column(u_to_key(best[j / ns]));
      carried[j] = (node >= 0 && node < nn) ? kids[(int64_t)node * ns + j % ns] : -1;
    }
    __syncthreads();
  }
  // the buckets: the carried children below the visible count, then the fresh buckets
  const int n_fresh = visible - covered > 0 ? visible - covered : 0;
  tree_candidates(cand, seen, a.rows, visible, carried, n_carried, covered, n_carried + n_fresh, a.cand_pow2);
  if (a.cache_keys) tree_gather_cached(cache + a.col_base[a.n_levels], cand, a.cand_pow2, keys);
  else if (!tree_gather(a, hd, pub + a.col_base[a.n_levels], cand, a.cand_pow2, keys)) return false;
  block_topk_fast(keys, a.cand_pow2, a.K, a.kp, best, tks, rst, bins, &hd.ok);
  return true;
}

template <typename T, int D, int GQ, bool TREE>
__device__ __forceinline__ void shared_reader(const SharedArgs& a, char* smem, int64_t i, int role) {
  using S = ReadShape<T, D, GQ>;
  constexpr int VEC = S::VEC, LPT = S::LPT, KPT = kShMaxRows / LSA_BLOCK;
  constexpr int PSTRIDE = GQ * (D + 2);
  ShHdr& hd = *(ShHdr*)smem;
  int32_t* first = (int32_t*)(smem + sh_picks_at());  // [kp]: a pick's first kept id
  int32_t* start = first + a.kp;                        // [kp + 1]: its first list slot
  char* region = smem + sh_region_at(a.kp);
  int32_t* ids = (int32_t*)region;                      // read: [chunk * span]
  ReadLds<D, GQ, kShMaxReaders>& rd = *(ReadLds<D, GQ, kShMaxReaders>*)(region + sh_rd_at(a.span));
  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1);
  const int K = a.K, rows = a.rows;
  const int64_t r = (uint32_t)i / (uint32_t)a.G;
  const int g = (int)((uint32_t)i % (uint32_t)a.G);
  const int64_t position = a.positions[r];
  const int64_t wstart = window_start_of(position, a.window);
  const int64_t n_win = position + 1 - wstart > 0 ? position + 1 - wstart : 0;
  const int64_t n_sink = a.sink < wstart ? a.sink : wstart;
  const int64_t t = r * a.row_tables;
  const int32_t* ends = a.ends + t * rows;

  // the query rows and the slot table row go out before the selection
  const T* qrow = (const T*)a.q + (r * a.Hq + (int64_t)g * GQ) * D;
  QueryRegs<T, D, GQ> qr;
  qr.load(qrow, a.scale_log2);
  const SlotRow map = slot_row_of(a.slots, r);
  const int32_t touched = touch_slot_lines(map, position, role, a.NR);

  uint64_t* best;
  const int32_t* ends_at;  // the span ends the placement reads (LDS or global)
  bool gave_up;
  if constexpr (!TREE) {
    int32_t* ends_l = (int32_t*)region;                             // [rows]
    best = (uint64_t*)(region + sh_best_at(rows));                  // [kp]
    uint64_t* cand = (uint64_t*)(region + sh_cand_at(rows, a.kp));  // [kp + 64]
    TopkScratch* tks = (TopkScratch*)(region + sh_topk_at(rows, a.kp));
    BinScratchWide* bins = (BinScratchWide*)((char*)tks + a16(sizeof(TopkScratch)));
    RadixState* rst = (RadixState*)((char*)bins + a16(sizeof(BinScratchWide)));
    for (int m = tid; m < rows; m += LSA_BLOCK) ends_l[m] = ends[m];
    ends_at = ends_l;
    // every wave polls its share of the row's keys (key m * 256 + tid in x[m]) until all of
    // them are written, every load of a round in flight together
    const uint64_t* pub = a.pub + r * a.n_cols;
    uint64_t x[KPT];
    int bad = 0;
    for (int it = 0;; ++it) {
      bool ok = true;
#pragma unroll
      for (int m = 0; m < KPT; ++m) {
        const int j = m * LSA_BLOCK + tid;
        x[m] = coherent_load_u64(pub + (j < rows ? j : 0));
        ok &= j >= rows || x[m] != 0;
      }
      if (__all(ok)) break;
      if (it >= a.spin_limit) {
        bad = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    DECODE_MARK(1);
#pragma unroll
    for (int m = 0; m < KPT; ++m) x[m] = m * LSA_BLOCK + tid < rows ? x[m] - 1 : 0;  // EMPTY past the table
    gave_up = block_gave_up(hd, bad);
    if (!gave_up) {
      // the K best keys, sorted (the select's top-K on the same keys)
      if (!topk_bins_regs<KPT, kTopBinsWide>(x, K, a.kp, best, cand, tks, bins)) topk_radix_regs<KPT>(x, K, a.kp, best, rst);
    }
  } else {
    const TreeLds L =
        tree_lds(a.cand_pow2, a.kp > a.beam_pow2 ? a.kp : a.beam_pow2, a.carry_cap, a.cache_keys ? a.n_cols : 0);
    best = (uint64_t*)(region + L.best);
    ends_at = ends;
    gave_up = !tree_walk(a, hd, region, r, t, position, best);
  }
  keep_live(touched);
  if (gave_up) {
    // no keys: this reader writes nothing but still arrives, so the counters reset; *status
    // tells the caller the launch's outputs are invalid
    if (tid == 0 && a.status) __hip_atomic_store(a.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (arrive_last(&a.rd_count[i], a.NR, &rd.flag)) shared_unit_done(a, hd, r);
    return;
  }
  DECODE_MARK(7);

  // each pick's kept range from the span ends, placed by one block scan, clipped at top_k
  constexpr int PPT = kShMaxPicks / LSA_BLOCK;
  int lo[PPT], cnt[PPT], mine = 0;
  int32_t eb[PPT], ee[PPT];
  bool okb[PPT];
#pragma unroll
  for (int p = 0; p < PPT; ++p) {  // every pick's two span ends in flight together
    const int j = PPT * tid + p;
    const int32_t b = j < K ? key_column(u_to_key(best[j])) : -1;
    okb[p] = b >= 0 && b < rows;
    eb[p] = okb[p] && b > 0 ? ends_at[b - 1] : 0;
    ee[p] = okb[p] ? ends_at[b] : 0;
  }
#pragma unroll
  for (int p = 0; p < PPT; ++p) {
    const int64_t l = eb[p] > a.sink ? eb[p] : a.sink, h = ee[p] < wstart ? ee[p] : wstart;
    lo[p] = (int)l;
    cnt[p] = okb[p] && h > l ? (int)(h - l) : 0;
    mine += cnt[p];
  }
  int total;
  int at = block_exclusive_sum(mine, hd.scan, &total);
  const int filled = total < a.top_k ? total : a.top_k;
#pragma unroll
  for (int p = 0; p < PPT; ++p) {
    const int j = PPT * tid + p;
    if (j < K) {
      first[j] = lo[p];
      start[j] = at < filled ? at : filled;
    }
    at += cnt[p];
  }
  if (tid == 0) {
    start[K] = filled;
    hd.filled = filled;
    if (g == 0 && role == 0) a.lengths[r] = filled + (int)(n_win + n_sink);
  }
  __syncthreads();  // picks placed; the selection phase's LDS is free from here
  DECODE_MARK(8);

  // the read: reader `role` takes a contiguous run of the list's tiles
  const int length = filled + (int)(n_win + n_sink);
  const int span = a.span, NR = a.NR;
  const int TT = (length + span - 1) / span;
  const int q_t = TT / NR, rem = TT % NR;
  const int t_lo = role * q_t + (role < rem ? role : rem);
  const int t_hi = t_lo + q_t + (role < rem ? 1 : 0);
  const int lo_s = t_lo * span, hi_s = min(length, t_hi * span);
  const int n_part = TT < NR ? TT : NR;
  int32_t* lrow = a.lists + r * (int64_t)a.W;
  const bool writer = g == 0;  // the shared list is written once, by kv-head 0's readers
  const int lp = lane % LPT;
  const T* kb = (const T*)a.k + r * a.kv_sb + g * a.kv_sh + lp * VEC;
  const T* vb = (const T*)a.v + r * a.kv_sb + g * a.kv_sh + lp * VEC;
  auto pick_of = [&](int s_) {  // the last pick whose first slot is <= s_
    int a_ = 0, b_ = K;
    while (b_ - a_ > 1) {
      const int m_ = (a_ + b_) >> 1;
      if (start[m_] <= s_) a_ = m_; else b_ = m_;
    }
    return a_;
  };
  if (writer) {  // the list's padding [length, W), shared out over the readers
    const int per = (a.W - length + NR - 1) / NR;
    const int p0 = length + role * per;
    const int p1 = min(p0 + per, a.W);
    for (int k = p0 + tid; k < p1; k += LSA_BLOCK) lrow[k] = -1;
  }
  AttnState<T, D, GQ> st;
  st.clear();
  bool fresh = true;
  for (int c_lo = lo_s; c_lo < hi_s; c_lo += kShChunkTiles * span) {
    const int c_hi = min(hi_s, c_lo + kShChunkTiles * span);
    const int n = c_hi - c_lo;
    for (int k = tid; k < n; k += LSA_BLOCK) {
      const int s_ = c_lo + k;
      int32_t id;
      if (s_ < filled) {
        const int j = pick_of(s_);
        id = first[j] + (s_ - start[j]);
      } else {
        id = tail_id(s_ - filled, wstart, n_win, n_sink);
      }
      id = map(id);
      ids[k] = id;
      if (writer) lrow[s_] = id;
    }
    __syncthreads();
    attend_tiles<T, D, GQ, true>(
        qr, kb, vb, a.kv_st, a.Tk, 0, n,
        [&](int jj) {
          const int32_t v_ = ids[jj < n ? jj : 0];
          return jj < n ? v_ : -1;
        },
        a.scale_log2, fresh, st);
    fresh = false;
    __syncthreads();  // ids are rewritten by the next chunk
  }

  DECODE_MARK(3);
  T* outp = (T*)a.out + (r * a.Hq + (int64_t)g * GQ) * D;
  float* parts = a.ws_part + i * (int64_t)NR * PSTRIDE;
  if (role < n_part) {
    finish_span<T, D, GQ>(rd, st, n_part == 1, outp, n_part > 1 ? parts + (int64_t)role * PSTRIDE : nullptr, 0);
  }
  DECODE_MARK(11);
  if (!arrive_last(&a.rd_count[i], NR, &rd.flag)) return;
  if (n_part > 1) {
    combine_partials<T, D, GQ>(rd, parts, n_part, outp, 0);
  } else if (n_part == 0) {  // nothing to read: zeros
    for (int k = tid; k < GQ * D; k += LSA_BLOCK) store_out<T>(outp + k, 0.0f);
  }
  DECODE_MARK(13);
  shared_unit_done(a, hd, r);
}

template <typename T, typename CT, int D, int GQ, bool TREE>
__global__ __launch_bounds__(LSA_BLOCK) void decode_shared_kernel(SharedArgs a) {
  extern __shared__ __align__(16) char smem[];
  const uint32_t nsel = (uint32_t)a.R * (uint32_t)a.S;  // the grid is < 2^31 workgroups (checked on the host)
  const uint32_t id = blockIdx.x;
  DECODE_TRACE_BEGIN();
  if (id < nsel) {
    shared_select<CT, D, TREE>(a, smem, id % (uint32_t)a.R, (int)(id / (uint32_t)a.R));
  } else {
    const uint32_t units = (uint32_t)a.R * (uint32_t)a.G;
    const uint32_t rid = id - nsel;  // readers: unit fastest, then role (low roles have work)
    shared_reader<T, D, GQ, TREE>(a, smem, rid % units, (int)(rid / units));
  }
  DECODE_TRACE_END();
}

// ------------------------------------------------------------------ host

template <typename T, typename CT, int D, bool TREE>
void launch_sh_gq(const SharedArgs& a, int gq, dim3 grid, size_t shmem, hipStream_t s) {
  switch (gq) {
    case 1: decode_shared_kernel<T, CT, D, 1, TREE><<<grid, LSA_BLOCK, shmem, s>>>(a); break;
    case 2: decode_shared_kernel<T, CT, D, 2, TREE><<<grid, LSA_BLOCK, shmem, s>>>(a); break;
    case 4: decode_shared_kernel<T, CT, D, 4, TREE><<<grid, LSA_BLOCK, shmem, s>>>(a); break;
    default: decode_shared_kernel<T, CT, D, 8, TREE><<<grid, LSA_BLOCK, shmem, s>>>(a); break;
  }
}

template <bool TREE>
void launch_sh(const SharedArgs& a, int dtype, bool bf16_table, int D, int gq, dim3 grid, size_t shmem,
               hipStream_t s) {
  if (dtype == LSA_BF16) {
    if (bf16_table) {
      if (D == 64) launch_sh_gq<bf16_t, bf16_t, 64, TREE>(a, gq, grid, shmem, s);
      else launch_sh_gq<bf16_t, bf16_t, 128, TREE>(a, gq, grid, shmem, s);
    } else {
      if (D == 64) launch_sh_gq<bf16_t, float, 64, TREE>(a, gq, grid, shmem, s);
      else launch_sh_gq<bf16_t, float, 128, TREE>(a, gq, grid, shmem, s);
    }
  } else {
    if (bf16_table) {
      if (D == 64) launch_sh_gq<_Float16, bf16_t, 64, TREE>(a, gq, grid, shmem, s);
      else launch_sh_gq<_Float16, bf16_t, 128, TREE>(a, gq, grid, shmem, s);
    } else {
      if (D == 64) launch_sh_gq<_Float16, float, 64, TREE>(a, gq, grid, shmem, s);
      else launch_sh_gq<_Float16, float, 128, TREE>(a, gq, grid, shmem, s);
    }
  }
}

inline size_t sh_read_lds(int D, int gq, int span) {
  if (D == 64) {
    switch (gq) {
      case 1: return sh_read_bytes<64, 1>(span);
      case 2: return sh_read_bytes<64, 2>(span);
      case 4: return sh_read_bytes<64, 4>(span);
      default: return sh_read_bytes<64, 8>(span);
    }
  }
  switch (gq) {
    case 1: return sh_read_bytes<128, 1>(span);
    case 2: return sh_read_bytes<128, 2>(span);
    case 4: return sh_read_bytes<128, 4>(span);
    default: return sh_read_bytes<128, 8>(span);
  }
}

// Readers per unit by default: about 24 (the list's tiles spread over CUs) but enough for
// ~512 workgroups in all when there are many units, never more tiles than a list holds.
constexpr int kShDefaultReaders = 24;
constexpr int kShSpread = 512;

inline int sh_readers(int64_t units, int span, int top_k, int window, int sink) {
  const int64_t tiles = ((int64_t)top_k + window + sink + span - 1) / span;
  int64_t nr = kShDefaultReaders;
  const int64_t spread = (kShSpread + units - 1) / units;
  if (spread < nr) nr = spread;
  if (tiles < nr) nr = tiles;
  if (nr < 1) nr = 1;
  return (int)nr;
}

// Word offset of the published keys (after the reader arrivals and the rows' unit counts).
inline int64_t sh_keys_at(int64_t R, int32_t G) { return (R * G + R + 63) / 64 * 64; }

inline size_t sh_scratch(int dtype, int64_t R, int32_t Hq, int32_t Hkv, int32_t D, int32_t top_k, int32_t window,
                  int32_t sink, int32_t readers) {
  if (R <= 0 || Hkv <= 0 || Hq < Hkv || Hq % Hkv) return 0;
  const int gq = Hq / Hkv;
  const int span = lsa_read_tile_tokens(dtype, D, gq);
  if (span <= 0) return 0;
  const int NR = readers > 0 ? readers : sh_readers(R * Hkv, span, top_k < 0 ? 0 : top_k, window < 0 ? 0 : window,
                                                    sink < 0 ? 0 : sink);
  return NR > 1 ? (size_t)(R * Hkv) * NR * (size_t)(gq * (D + 2)) * sizeof(float) : 0;
}

// Checks both entry points share; fills the K/V, table, list and hand-off fields of `a`.
inline int sh_common(const char* who, SharedArgs& a, const void* q, const void* k, const void* v, int dtype, int64_t R,
              int64_t Tk, int32_t Hq, int32_t Hkv, int32_t D, int64_t kv_batch_stride, int64_t kv_token_stride,
              int64_t kv_head_stride, const float* index_queries, const void* centroids, const int32_t* ends,
              int32_t table_flags, int32_t rows, int64_t row_tables, int score_mode, const int32_t* positions,
              const lsa_slot_map* slots, int32_t cluster_block_size, int32_t block_buckets, int32_t top_p,
              int32_t window, int32_t sink, int32_t top_k, float scale, int32_t readers, int32_t* counters,
              int32_t* lists, int32_t* lengths, void* out, int32_t* status) {
  LSA_REQUIRE(q && k && v && index_queries && centroids && ends && positions && lists && lengths && out && counters,
              LSA_ERR_NULL, "%s: NULL pointer", who);
  SlotMap sm;
  LSA_TRY(check_slots(who, slots, &sm));
  LSA_REQUIRE(dtype == LSA_BF16 || dtype == LSA_F16, LSA_ERR_DTYPE, "%s: bf16 or fp16 K/V, got dtype %d", who,
              dtype);
  LSA_REQUIRE(D == 64 || D == 128, LSA_ERR_SHAPE, "%s: head dim %d not in {64, 128}", who, D);
  LSA_REQUIRE(Hq >= 1 && Hkv >= 1 && Hq % Hkv == 0, LSA_ERR_SHAPE, "%s: Hq %d must group onto Hkv %d", who, Hq, Hkv);
  const int gq = Hq / Hkv;
  LSA_REQUIRE(gq == 1 || gq == 2 || gq == 4 || gq == 8, LSA_ERR_SHAPE, "%s: group size %d not in {1,2,4,8}", who,
              gq);
  LSA_REQUIRE(score_mode == LSA_SCORE_BF16 || score_mode == LSA_SCORE_F32, LSA_ERR_DTYPE, "%s: bad score mode", who);
  LSA_REQUIRE(rows >= 1 && row_tables >= 0, LSA_ERR_SHAPE, "%s: bad table sizes", who);
  LSA_REQUIRE(R >= 0 && Tk >= 0 && Tk <= 0x7FFFFFFF, LSA_ERR_SHAPE, "%s: bad sizes", who);
  LSA_REQUIRE(top_p >= 1 && window >= 0 && sink >= 0 && top_k >= 0, LSA_ERR_SHAPE,
              "%s: top_p >= 1, window/sink/top_k >= 0", who);
  LSA_REQUIRE((table_flags & ~(LSA_TABLE_SPANS | LSA_TABLE_BLOCK_VISIBLE)) == 0 && (table_flags & LSA_TABLE_SPANS),
              LSA_ERR_SHAPE, "%s: span tables (LSA_TABLE_SPANS, optionally LSA_TABLE_BLOCK_VISIBLE), got flags %d",
              who, table_flags);
  LSA_REQUIRE(!(table_flags & LSA_TABLE_BLOCK_VISIBLE) || cluster_block_size >= 1, LSA_ERR_SHAPE,
              "%s: cluster_block_size must be >= 1", who);
  LSA_REQUIRE((int64_t)top_k + window + sink <= 0x7FFFFFFF, LSA_ERR_SHAPE, "%s: list too wide", who);
  const uintptr_t mis = ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)centroids) & 15;
  LSA_REQUIRE(mis == 0 && ((uintptr_t)index_queries & 15) == 0, LSA_ERR_ALIGN,
              "%s: q/k/v/centroids/index queries must be 16-byte aligned", who);
  LSA_REQUIRE(kv_batch_stride >= 0 && kv_token_stride >= D && kv_head_stride >= D, LSA_ERR_SHAPE,
              "%s: K/V strides must leave rows of %d elements apart", who, D);
  LSA_REQUIRE(((kv_batch_stride | kv_token_stride | kv_head_stride) * 2) % 16 == 0, LSA_ERR_ALIGN,
              "%s: K/V strides must keep rows 16-byte aligned", who);
  LSA_REQUIRE(readers >= 0 && readers <= kShMaxReaders, LSA_ERR_SHAPE, "%s: readers in [0, %d], got %d", who,
              kShMaxReaders, readers);
  a.q = q; a.k = k; a.v = v; a.out = out;
  a.R = R; a.G = Hkv; a.Hq = Hq;
  a.Tk = Tk; a.kv_sb = kv_batch_stride; a.kv_st = kv_token_stride; a.kv_sh = kv_head_stride;
  a.idx_q = index_queries; a.centroids = centroids; a.ends = ends;
  a.vends = (table_flags & LSA_TABLE_BLOCK_VISIBLE) ? nullptr : ends;
  a.rows = rows; a.row_tables = row_tables; a.positions = positions;
  a.cluster_block = cluster_block_size; a.block_buckets = block_buckets;
  a.window = window; a.sink = sink; a.top_k = top_k; a.W = top_k + window + sink;
  a.scale_log2 = scale * kLog2e;
  a.spin_limit = decode_debug().spin_limit > 0 ? decode_debug().spin_limit : 1 << 22;
  a.skip_publish = decode_debug().skip_publish;
  a.lists = lists; a.lengths = lengths; a.status = status;
  a.slots = sm;
  a.n_levels = 0;
  a.cache_keys = 0;
  return LSA_OK;
}

// The rest of both entry points once `a` holds the selection's fields (K, kp, n_cols):
// reader count, LDS (sel_lds: the selection phase's reader region), grid, buffers, launch.
template <bool TREE>
int sh_finish(const char* who, SharedArgs& a, int dtype, int32_t D, int score_mode, int32_t select_splits,
              int32_t readers, size_t sel_lds, int32_t* counters, int64_t n_counters, int64_t need_counters,
              void* scratch, size_t scratch_bytes, void* stream) {
  const int64_t units = a.R * a.G;
  if (units == 0) return LSA_OK;
  const int gq = a.Hq / a.G;
  const int span = lsa_read_tile_tokens(dtype, D, gq);
  LSA_REQUIRE(span > 0, LSA_ERR_SHAPE, "%s: no read tile for D=%d group=%d", who, D, gq);
  const int NR = readers > 0 ? readers : sh_readers(units, span, a.top_k, a.window, a.sink);
  const int64_t dflt = (a.n_cols + 63) / 64 < 256 ? (a.n_cols + 63) / 64 : 256;
  const int64_t S = select_splits > 0 ? select_splits : dflt;
  LSA_REQUIRE(S >= 1 && S <= 256 && S <= a.n_cols, LSA_ERR_SHAPE,
              "%s: select splits in [1, min(256, columns %lld)], got %lld", who, (long long)a.n_cols, (long long)S);
  const int64_t cs = (a.n_cols + S - 1) / S;
  const size_t rd = sh_read_lds(D, gq, span);
  const size_t reader_lds = sh_region_at(a.kp) + (sel_lds > rd ? sel_lds : rd);
  const size_t select_lds = sizeof(uint64_t) * (size_t)cs;
  const size_t lds = reader_lds > select_lds ? reader_lds : select_lds;
  LSA_REQUIRE(lds <= kShMaxLds, LSA_ERR_SHAPE, "%s: %zu bytes of LDS exceed %zu (fewer buckets, nodes or picks)",
              who, lds, kShMaxLds);
  const int64_t grid = a.R * S + units * NR;
  LSA_REQUIRE(grid <= 0x7FFFFFFF && units < (1ll << 31), LSA_ERR_SHAPE, "%s: too many workgroups", who);
  LSA_REQUIRE(need_counters > 0 && n_counters >= need_counters, LSA_ERR_WORKSPACE, "%s: %lld counters < %lld", who,
              (long long)n_counters, (long long)need_counters);
  const size_t need = sh_scratch(dtype, a.R, a.Hq, a.G, D, a.top_k, a.window, a.sink, NR);
  LSA_REQUIRE(need == 0 || (scratch && scratch_bytes >= need), LSA_ERR_WORKSPACE, "%s: scratch %zu < %zu bytes", who,
              scratch_bytes, need);
  LSA_REQUIRE(((uintptr_t)scratch % 16) == 0 && ((uintptr_t)counters % 8) == 0, LSA_ERR_ALIGN,
              "%s: scratch must be 16-byte and counters 8-byte aligned", who);
  a.S = (int)S; a.cs = (int)cs; a.span = span; a.NR = NR;
  a.rd_count = counters;
  a.done = counters + units;
  a.pub = (uint64_t*)(counters + sh_keys_at(a.R, a.G));
  a.ws_part = need ? (float*)scratch : nullptr;
  const dim3 g3((unsigned)grid);
  hipStream_t s = (hipStream_t)stream;
  const bool bf16_table = score_mode == LSA_SCORE_BF16;
  launch_sh<TREE>(a, dtype, bf16_table, D, gq, g3, lds, s);
  LSA_LAUNCHED(who);
  return LSA_OK;
}

// The most candidates a tree level scores (the beam select's bound): at the start level its
// made nodes; below, the carried children plus the open nodes; at the buckets the carried
// children plus the fresh buckets.
inline int64_t tree_most(int levels, const int32_t* n_nodes, int rows, int node_size, int node_block, int beam) {
  const int64_t carry = (int64_t)beam * node_size;
  int64_t most = n_nodes[levels - 1] > node_block - 1 ? n_nodes[levels - 1] : node_block - 1;
  for (int l = 0; l < levels; ++l) {
    const int64_t below = l == 0 ? rows : n_nodes[l - 1];
    const int64_t past = below - (int64_t)n_nodes[l] * node_size;
    int64_t open = past > node_block - 1 ? past : node_block - 1;
    open = open < below ? open : below;
    most = carry + open > most ? carry + open : most;
  }
  return most;
}

}  // namespace shared
}  // namespace lsa
