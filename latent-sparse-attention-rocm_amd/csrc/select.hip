// Selection kernels for gfx950: canonical scoring, the whole-path listing, best-first
// top-k, unpack, the rank-order expansion, the fused flat select (score + top-k +
// expansion, split over workgroups for decode) and the two-level tree select.
//
// Reference behaviour restated: pipeline.py:184-316 (visible_counts, best_first_keys,
// _production_scores, flat_select[_reference]), select_fused.py:52-280
// (select_topk_scores, expand_in_order_from_keys), _tree.py:318-373 (_beam_pick_rows) with
// _tree.py:100-142 (_growth_replay) for one node level.
#include "lsa_abi_common.h"
#include "lsa_screen_dev.h"
#include "lsa_select_dev.h"

using namespace lsa;

namespace {

constexpr int kMaxLdsKeys = 6144;  // u64 keys a workgroup holds in LDS (48 KiB, under the 64 KiB default)
constexpr size_t kMaxDynLds = 56 * 1024;  // dynamic LDS of a select workgroup, beside ~6 KiB of static state

// ------------------------------------------------------------------ visible counts

__global__ void visible_counts_kernel(const int32_t* positions, int64_t R, int G, int rows, int cluster_block,
                                      int block_buckets, const int32_t* ends, int64_t row_tables,
                                      int64_t group_tables, int32_t* counts) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= R * G) return;
  const int64_t r = i / G, g = i % G;
  const int32_t* e = ends ? ends + (r * row_tables + g * group_tables) * rows : nullptr;
  counts[i] = visible_count(positions[r], rows, cluster_block, block_buckets, e);
}

// ------------------------------------------------------------------ scores

template <typename QT, typename CT, int SPAN>
__global__ __launch_bounds__(LSA_BLOCK) void score_rows_kernel(const QT* q, int G, const CT* cent, int N,
                                                               int64_t row_tables, int64_t group_tables,
                                                               bool bf16_mode, float* out) {
  constexpr int D = 16 * SPAN;
  const int64_t i = blockIdx.x;
  const int64_t r = i / G, g = i % G;
  const int p = threadIdx.x & 15, grp = threadIdx.x >> 4;
  float qs[SPAN];
  load_query_slice<QT, SPAN>(q + i * D, p, bf16_mode, qs);
  const CT* tab = cent + (r * row_tables + g * group_tables) * (int64_t)N * D;
  const int c = blockIdx.y * (LSA_BLOCK / 16) + grp;
  if (c < N) {
    const float s = canonical_score<CT, SPAN>(qs, tab + (int64_t)c * D, p);
    if (p == 0) out[i * N + c] = s;
  }
}

// ------------------------------------------------------------------ listing / unpack

__global__ void pack_listing_kernel(const float* scores, const int32_t* counts, int64_t R, int N, int64_t* keys) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= R * N) return;
  const int64_t r = i / N;
  const int c = (int)(i % N);
  keys[i] = c < counts[r] ? pack_key(scores[i], c) : kEmpty;
}

__global__ void unpack_kernel(const int64_t* keys, int64_t n, int32_t* ids) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < n) ids[i] = key_column(keys[i]);
}

// ------------------------------------------------------------------ top-k

struct KeySource {  // best_first_keys: existing keys, optional listing counts
  const int64_t* keys;
  const int32_t* counts;
  int W;
  __device__ uint64_t get(int64_t row, int i) const {
    if (counts && i >= counts[row]) return 0;
    return key_to_u(keys[row * W + i]);
  }
};

struct ScoreSource {  // select_topk_scores: pack from fp32 scores, EMPTY past length
  const float* scores;
  const int32_t* lengths;
  int W;
  __device__ uint64_t get(int64_t row, int i) const {
    if (i >= lengths[row]) return 0;
    return key_to_u(pack_key(scores[row * W + i], i));
  }
};

// One row per workgroup: radix-select the k-th best key, collect the k best, bitonic
// sort them descending, write k_out keys (EMPTY past k). LDS mode keeps the row in LDS.
template <typename Src, bool LDS_ROW>
__global__ __launch_bounds__(LSA_BLOCK) void topk_kernel(Src src, int W, int k, int kp, int k_out, int64_t* out) {
  extern __shared__ uint64_t smem[];
  __shared__ RadixState st;
  const int64_t row = blockIdx.x;
  uint64_t* buf = smem;
  uint64_t* row_keys = smem + kp;
  if (LDS_ROW) {
    for (int i = threadIdx.x; i < W; i += LSA_BLOCK) row_keys[i] = src.get(row, i);
    __syncthreads();
  }
  auto get = [&](int i) -> uint64_t { return LDS_ROW ? row_keys[i] : src.get(row, i); };
  radix_select(get, W, k, &st);
  radix_collect(get, W, k, &st, buf);
  for (int i = k + threadIdx.x; i < kp; i += LSA_BLOCK) buf[i] = 0;
  __syncthreads();
  bitonic_sort_desc(buf, kp);
  for (int i = threadIdx.x; i < k_out; i += LSA_BLOCK) out[row * k_out + i] = i < k ? u_to_key(buf[i]) : kEmpty;
}

// ------------------------------------------------------------------ expansion

template <bool KEYS>
__global__ __launch_bounds__(LSA_BLOCK) void expand_kernel(const void* picks, int G, int P, const int32_t* members,
                                                           int rows, int cap, int64_t row_tables,
                                                           int64_t group_tables, const int32_t* positions,
                                                           SlotMap slots, int window, int sink, int top_k,
                                                           int32_t* lists, int32_t* lengths) {
  extern __shared__ int32_t pk[];
  __shared__ int scan[LSA_WAVES];
  const int64_t i = blockIdx.x;
  const int64_t r = i / G, g = i % G;
  for (int j = threadIdx.x; j < P; j += LSA_BLOCK) {
    pk[j] = KEYS ? key_column(((const int64_t*)picks)[i * P + j]) : ((const int32_t*)picks)[i * P + j];
  }
  __syncthreads();
  const int32_t* tab = members + (r * row_tables + g * group_tables) * (int64_t)rows * cap;
  const int width = top_k + window + sink;
  const int len = expand_walk(pk, P, tab, rows, cap, positions[r], window, sink, top_k, lists + i * width, width,
                              scan, nullptr, slot_row_of(slots, r));
  if (threadIdx.x == 0) lengths[i] = len;
}

// ------------------------------------------------------------------ fused flat select

struct FlatArgs {
  int64_t R;
  int G;
  int rows, cap;
  int64_t row_tables, group_tables;
  const void* centroids;
  const int32_t* members;
  const int32_t* ends;
  const int32_t* positions;
  int cluster_block, block_buckets;
  int K, kp;          // picks kept (min(top_p, rows)) and its power of two
  int window, sink, top_k;
  int S, cs;          // splits and columns per split
  int stage;          // 1: the list row is assembled in LDS after keys and picks
  int wide_stage;     // span tables with K > 64: the row is staged in the (dead) keys region after the picks
  int screen;         // one split, bf16 tables that fit screen_topk: matrix-core screen + exact re-score
  int spans;          // bucket row j holds exactly ids ends[j - 1] .. ends[j] - 1 (ends[-1] = 0)
  const int32_t* vends;  // the ends that decide visibility (nullptr: the closed-block rule)
  uint64_t* ws_keys;  // [R*G, rows] every column's key (S > 1)
  int* ws_count;      // [R*G] arrival counters (S > 1)
  SlotMap slots;      // a paged cache's slot table (table == nullptr: none)
  int32_t* lists;
  int32_t* lengths;
};

// The rank-order expansion of one row's picks pk[0..K) (in LDS) into its read list and
// length: span tables from the picks' span ends, member tables by the walk over member
// rows (staged in LDS after the keys when a.stage). Every thread calls it.
__device__ __forceinline__ void expand_row(const FlatArgs& a, const int32_t* pk, int64_t t, const int32_t* ends,
                                           int64_t position, int64_t i, int* scan) {
  extern __shared__ uint64_t smem[];
  const int width = a.top_k + a.window + a.sink;
  const SlotRow map = slot_row_of(a.slots, i / a.G);
  int len;
  if (a.spans && a.K <= LSA_WAVE) {  // span tables: kept ids from the picks' span ends, no member rows
    __shared__ int span_lds[2 * LSA_WAVE + 1];
    len = expand_spans(pk, a.K, ends, a.rows, position, a.window, a.sink, a.top_k, a.lists + i * width, width,
                       span_lds, map);
  } else if (a.spans) {  // more picks: one per-thread run of picks each, one block scan
    int32_t* stage = a.wide_stage ? (int32_t*)((char*)smem + ((4 * (size_t)a.K + 15) & ~(size_t)15)) : nullptr;
    len = a.K <= 4 * LSA_BLOCK
              ? expand_spans_wide<4>(pk, a.K, ends, a.rows, position, a.window, a.sink, a.top_k, a.lists + i * width,
                                     width, stage, scan, map)
              : expand_spans_wide<16>(pk, a.K, ends, a.rows, position, a.window, a.sink, a.top_k,
                                      a.lists + i * width, width, stage, scan, map);
  } else {
    const int32_t* tab = a.members + t * a.rows * (int64_t)a.cap;
    int32_t* stage = a.stage ? (int32_t*)(smem + ((a.rows + a.kp + 1) & ~1)) : nullptr;  // 16-byte aligned
    len = expand_walk(pk, a.K, tab, a.rows, a.cap, position, a.window, a.sink, a.top_k, a.lists + i * width, width,
                      scan, stage, map);
  }
  if (threadIdx.x == 0) a.lengths[i] = len;
}

// grid (R*G, S). Split s scores columns [s*cs, (s+1)*cs) of its table in one batch of
// loads (query slice, centroid rows and the columns' span ends together); with S > 1 it
// publishes the keys and the last split to arrive takes every column's key from the
// workspace. That workgroup selects the K best keys, sorted, and expands the picks into
// the read list in rank order (reference pipeline.py:248-316, select_fused.py:52-280).
// Four waves a SIMD (128 VGPRs, a few spilled): with one workgroup per row, the prefill's
// 4096 rows are latency-bound and the fourth resident workgroup a CU hides more of it
// (0.22 -> 0.20 ms for the 32k prefill select; the 8-row decode select is unchanged).
template <typename QT, typename CT, int SPAN>
__global__ __launch_bounds__(LSA_BLOCK) __attribute__((amdgpu_waves_per_eu(4, 4))) void select_flat_kernel(
    const QT* q, bool bf16_mode, FlatArgs a) {
  constexpr int D = 16 * SPAN;
  extern __shared__ uint64_t smem[];
  __shared__ RadixState st;
  __shared__ TopkScratch tks;
  __shared__ BinScratchWide bins;
  __shared__ int scan[LSA_WAVES];
  __shared__ int flag;
  uint64_t* keys = smem;            // [rows]
  uint64_t* best = smem + a.rows;   // [kp]
  const int64_t i = blockIdx.x;
  const int s = blockIdx.y;
  const int64_t r = i / a.G, g = i % a.G;
  const int64_t position = a.positions[r];
  const int64_t t = r * a.row_tables + g * a.group_tables;
  const CT* cent = (const CT*)a.centroids + t * a.rows * (int64_t)D;
  const int32_t* ends = a.ends ? a.ends + t * a.rows : nullptr;
  const int32_t* vends = a.vends ? a.vends + t * a.rows : nullptr;
  const int c0 = s * a.cs;
  const int c1 = min(c0 + a.cs, a.rows);
  const int n_local = c1 > c0 ? c1 - c0 : 0;
  const int vis = vends ? 0 : visible_closed(position, a.rows, a.cluster_block, a.block_buckets);
  const int64_t lim = position + 1;

  float qs[SPAN];
  load_query_slice<QT, SPAN>(q + i * D, threadIdx.x & 15, bf16_mode, qs);
  int32_t* pk = (int32_t*)keys;
  if constexpr (__is_same(CT, bf16_t) && SPAN >= 2 && SPAN <= 8) {
    if (a.screen) {  // the whole table on the matrix cores, exact (screen_topk)
      ScreenLds& scr = *(ScreenLds*)smem;
      uint64_t* sbest = (uint64_t*)((char*)smem + sizeof(ScreenLds));
      // span ends are nondecreasing: the visible rows are a prefix, counted once
      __shared__ int vis_lds[2 * LSA_WAVES];
      const int nvis = vends ? visible_count_block(position, a.rows, vends, vis_lds) : vis;
      screen_topk<D, 2>(
          qs, cent, a.rows, [](int j) { return j; }, [&](int j) { return j < nvis; }, a.K, a.kp, sbest, scr);
      for (int j = threadIdx.x; j < a.K; j += LSA_BLOCK) pk[j] = key_column(u_to_key(sbest[j]));
      __syncthreads();
      expand_row(a, pk, t, ends, position, i, scan);
      return;
    }
  }
  score_keys<CT, SPAN>(
      qs, cent, D, n_local, [&](int j) { return c0 + j; },
      [&](int j) { return vends ? (int64_t)vends[c0 + j] <= lim : c0 + j < vis; }, keys + c0);

  if (a.S > 1) {
    __syncthreads();
    uint64_t* mine = a.ws_keys + i * (int64_t)a.rows;
    for (int j = threadIdx.x; j < n_local; j += LSA_BLOCK) coherent_store_u64(mine + c0 + j, keys[c0 + j]);
    if (!arrive_last(&a.ws_count[i], a.S, &flag)) return;
    for (int jb = 0; jb < a.rows; jb += 16 * LSA_BLOCK) {  // 16 coherent loads in flight per thread
      uint64_t v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int j = jb + u * LSA_BLOCK + threadIdx.x;
        v[u] = coherent_load_u64(mine + (j < a.rows ? j : 0));
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int j = jb + u * LSA_BLOCK + threadIdx.x;
        if (j < a.rows) keys[j] = v[u];
      }
    }
  }
  __syncthreads();
  block_topk_any(keys, a.rows, a.K, a.kp, best, &tks, &st, &bins);
  for (int j = threadIdx.x; j < a.K; j += LSA_BLOCK) pk[j] = key_column(u_to_key(best[j]));
  __syncthreads();
  expand_row(a, pk, t, ends, position, i, scan);
}

// ------------------------------------------------------------------ two-level tree select

constexpr int kSeenBits = 8192;  // buckets a tree table may hold for the LDS dedup bitmap

struct TreeArgs {
  int64_t R;
  int G;
  const void* node_centroids;
  const int32_t* children;
  int n_nodes, node_size;
  const void* centroids;
  const int32_t* members;
  const int32_t* ends;
  int rows, cap;
  int64_t row_tables, group_tables;
  const int32_t* positions;
  int cluster_block, block_buckets;
  int node_block, beam, top_p;
  int nodes_pow2, beam_pow2, cand_cap, cand_pow2, top_pow2;
  int window, sink, top_k;
  int spans;  // bucket row j holds exactly ids ends[j - 1] .. ends[j] - 1 (ends[-1] = 0)
  const int32_t* vends;  // the ends that decide visibility (nullptr: the closed-block rule)
  int screen1, screen0;  // bf16 tables that fit screen_topk: node / bucket level on the matrix cores
  SlotMap slots;         // a paged cache's slot table (table == nullptr: none)
  int32_t* lists;
  int32_t* lengths;
};

template <typename QT, typename CT, int SPAN>
__global__ __launch_bounds__(LSA_BLOCK) void select_tree_kernel(const QT* q, bool bf16_mode, TreeArgs a) {
  constexpr int D = 16 * SPAN;
  extern __shared__ uint64_t smem[];
  __shared__ RadixState st;
  __shared__ TopkScratch tks;
  __shared__ BinScratch bins;
  __shared__ int scan[LSA_WAVES];
  __shared__ ScreenLds scr;
  uint64_t* keys = smem;                    // [max(nodes_pow2, cand_pow2)]
  uint64_t* best = keys + max(a.nodes_pow2, a.cand_pow2);  // [max(beam_pow2, top_pow2)]
  int32_t* cand = (int32_t*)(best + max(a.beam_pow2, a.top_pow2));  // [cand_cap]
  const int64_t i = blockIdx.x;
  const int64_t r = i / a.G, g = i % a.G;
  const int64_t position = a.positions[r];
  const int64_t t = r * a.row_tables + g * a.group_tables;
  const int p = threadIdx.x & 15, grp = threadIdx.x >> 4;
  float qs[SPAN];
  load_query_slice<QT, SPAN>(q + i * D, p, bf16_mode, qs);

  // the row's growth (reference _tree.py:100-142 with one level, page = the row's visible
  // count): nodes are made from whole blocks of node_block visible buckets, so the first
  // `covered` buckets lie under the made nodes [0, made) and [covered, visible) are fresh
  __shared__ int vis_lds[2 * LSA_WAVES];
  const int visible = max(0, a.vends ? visible_count_block(position, a.rows, a.vends + t * a.rows, vis_lds)
                                     : visible_count(position, a.rows, a.cluster_block, a.block_buckets, nullptr));
  const int covered = min(visible / a.node_block * a.node_block, a.n_nodes * a.node_size);
  const int made = covered / a.node_size;

  // level 1: the made nodes, the best `beam` (a tie to the lower node); the rest are EMPTY
  const CT* ncent = (const CT*)a.node_centroids + t * (int64_t)a.n_nodes * D;
  const int beam = min(a.beam, a.n_nodes);
  bool done1 = false;
  if constexpr (__is_same(CT, bf16_t) && SPAN >= 2 && SPAN <= 8) {
    if (a.screen1) {
      screen_topk<D, 2>(
          qs, ncent, a.n_nodes, [](int j) { return j; }, [&](int j) { return j < made; }, beam, a.beam_pow2, best,
          scr);
      done1 = true;
    }
  }
  if (!done1) {
    score_slice_keys<CT, SPAN>(qs, ncent, D, 0, a.n_nodes, made, keys);
    __syncthreads();
    block_topk_any(keys, a.n_nodes, beam, a.beam_pow2, best, &tks, &st, &bins);
  }

  // level 0 candidates: the kept nodes' children (only visible buckets), then the fresh
  // buckets [covered, visible)
  const int n_fresh = max(0, visible - covered);
  const int n_kids = beam * a.node_size;
  const int n_cand = n_kids + n_fresh;
  const int32_t* kids = a.children + t * (int64_t)a.n_nodes * a.node_size;
  auto candidate = [&](int j) -> int32_t {
    int32_t c = -1;
    if (j < n_kids) {
      const int node = key_column(u_to_key(best[j / a.node_size]));
      if (node >= 0) c = kids[(int64_t)node * a.node_size + j % a.node_size];
    } else if (j < n_cand) {
      c = covered + (j - n_kids);
    }
    return (c >= 0 && c < visible) ? c : -1;
  };
  // every candidate bucket once (the order does not matter: a key carries its column)
  if (a.rows <= kSeenBits) {  // an LDS bitmap over bucket ids: the first lane to set a bit keeps it
    __shared__ uint32_t seen[kSeenBits / 32];
    for (int x = threadIdx.x; x < (a.rows + 31) / 32; x += LSA_BLOCK) seen[x] = 0;
    __syncthreads();
    for (int j = threadIdx.x; j < a.cand_pow2; j += LSA_BLOCK) {
      const int32_t c = candidate(j);
      const uint32_t bit = 1u << (c & 31);
      cand[j] = (c >= 0 && !(atomicOr(&seen[c >> 5], bit) & bit)) ? c : -1;
    }
  } else {  // sort the ids: equal ids adjacent, keep the first
    for (int j = threadIdx.x; j < a.cand_pow2; j += LSA_BLOCK) {
      const int32_t c = candidate(j);
      keys[j] = c >= 0 ? (uint64_t)c + 1 : 0;  // id + 1, 0 = none
    }
    __syncthreads();
    bitonic_sort_desc(keys, a.cand_pow2);
    for (int j = threadIdx.x; j < a.cand_pow2; j += LSA_BLOCK) {
      const uint64_t v = keys[j];
      cand[j] = (v != 0 && (j == 0 || keys[j - 1] != v)) ? (int32_t)(v - 1) : -1;
    }
  }
  __syncthreads();
  const CT* bcent = (const CT*)a.centroids + t * (int64_t)a.rows * D;
  const int k = min(a.top_p, a.cand_pow2);
  bool done0 = false;
  if constexpr (__is_same(CT, bf16_t) && SPAN >= 2 && SPAN <= 8) {
    if (a.screen0) {
      screen_topk<D, 2>(
          qs, bcent, a.cand_pow2, [&](int j) { return cand[j]; }, [](int) { return true; }, k, a.top_pow2, best,
          scr);
      done0 = true;
    }
  }
  if (!done0) {
    score_keys<CT, SPAN>(qs, bcent, D, a.cand_pow2, [&](int j) { return cand[j]; }, keys);
    __syncthreads();
    block_topk_any(keys, a.cand_pow2, k, a.top_pow2, best, &tks, &st, &bins);
  }
  for (int j = threadIdx.x; j < a.top_p; j += LSA_BLOCK) cand[j] = j < k ? key_column(u_to_key(best[j])) : -1;
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

// ------------------------------------------------------------------ index queries / centroids

// V consecutive elements of a row as floats (one 4 V-byte or 2 V-byte load).
template <typename QT, int V> struct RowVec;
template <typename QT> struct RowVec<QT, 1> {
  static __device__ __forceinline__ void load(const QT* p, float* f) { f[0] = elem<QT>::load(p, 0); }
};
template <> struct RowVec<float, 4> {
  static __device__ __forceinline__ void load(const float* p, float* f) {
    const float4 x = *(const float4*)p;
    f[0] = x.x; f[1] = x.y; f[2] = x.z; f[3] = x.w;
  }
};
template <> struct RowVec<bf16_t, 4> {
  static __device__ __forceinline__ void load(const bf16_t* p, float* f) {
    const uint2 x = *(const uint2*)p;
    f[0] = __uint_as_float(x.x << 16); f[1] = __uint_as_float(x.x & 0xFFFF0000u);
    f[2] = __uint_as_float(x.y << 16); f[3] = __uint_as_float(x.y & 0xFFFF0000u);
  }
};
template <> struct RowVec<_Float16, 4> {
  static __device__ __forceinline__ void load(const _Float16* p, float* f) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 x = *(const h4*)p;
    f[0] = (float)x[0]; f[1] = (float)x[1]; f[2] = (float)x[2]; f[3] = (float)x[3];
  }
};

// One thread per V dims of an output row (b, chunk, kv-head): the fp32 sum over the
// chunk's tokens and, within a token, the group's heads in order (the canonical order),
// then one division. The (token, head) rows are walked in batches of 16 whose loads are
// all in flight before the batch's adds.
template <typename QT, int V>
__global__ void index_queries_kernel(const QT* q, int64_t B, int64_t T, int Hq, int Hkv, int D, int chunk,
                                     float* out) {
  const int64_t C = T / chunk;
  const int DV = D / V;
  const int64_t n = B * C * Hkv * DV;
  const int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const int dv = (int)(idx % DV);
  const int g = (int)((idx / DV) % Hkv);
  const int64_t c = (idx / ((int64_t)DV * Hkv)) % C;
  const int64_t b = idx / ((int64_t)DV * Hkv * C);
  const int G = Hq / Hkv;
  const QT* base = q + ((b * T + c * chunk) * Hq + (int64_t)g * G) * D + dv * V;
  const int64_t tstride = (int64_t)Hq * D;
  const int rows = chunk * G;  // (token, head) rows, token-major
  constexpr int NB = 16;
  float acc[V];
#pragma unroll
  for (int e = 0; e < V; ++e) acc[e] = 0.0f;
  for (int k0 = 0; k0 < rows; k0 += NB) {
    float x[NB][V];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int k = k0 + j < rows ? k0 + j : rows - 1;  // clamped: every load in bounds
      const int t = k / G, h = k - t * G;
      RowVec<QT, V>::load(base + t * tstride + (int64_t)h * D, x[j]);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (k0 + j < rows) {
#pragma unroll
        for (int e = 0; e < V; ++e) acc[e] += x[j][e];
      }
    }
  }
  const float cnt = (float)(chunk * G);
#pragma unroll
  for (int e = 0; e < V; ++e) out[idx * V + e] = acc[e] / cnt;
}

template <typename KT>
__global__ __launch_bounds__(LSA_BLOCK) void centroids_kernel(const KT* keys, int64_t tokens, int64_t token_stride,
                                                              int64_t batch_stride, int kv_heads, int D,
                                                              const int32_t* members, int rows, int cap,
                                                              int mode, float* out_f32, uint16_t* out_bf16) {
  __shared__ float sums[512];
  __shared__ float norm;
  const int64_t bucket = blockIdx.x;
  const int64_t table = bucket / rows;
  const KT* kb = keys + (table / kv_heads) * batch_stride + (table % kv_heads) * (int64_t)D;
  const int32_t* m = members + bucket * cap;
  int count = 0;
  for (int j = 0; j < cap; ++j) count += (m[j] >= 0 && m[j] < tokens) ? 1 : 0;
  for (int d = threadIdx.x; d < D; d += LSA_BLOCK) {
    float acc = 0.0f;
    for (int j = 0; j < cap; ++j) {
      const int32_t id = m[j];
      if (id >= 0 && id < tokens) acc += elem<KT>::load(kb, (int64_t)id * token_stride + d);
    }
    sums[d] = acc;
  }
  __syncthreads();
  if (mode == LSA_CENTROID_NORMALIZED && threadIdx.x == 0) {
    double sq = 0.0;
    for (int d = 0; d < D; ++d) sq += (double)sums[d] * (double)sums[d];
    norm = fmaxf((float)sqrt(sq), 1e-12f);
  }
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += LSA_BLOCK) {
    float c;
    if (mode == LSA_CENTROID_NORMALIZED) c = sums[d] / norm;
    else if (mode == LSA_CENTROID_SUM) c = sums[d];
    else c = count > 0 ? sums[d] / (float)count : 0.0f;
    out_f32[bucket * D + d] = c;
    if (out_bf16) out_bf16[bucket * D + d] = f32_to_bf16(c);
  }
}

}  // namespace

extern "C" int lsa_visible_counts(const int32_t* positions, int64_t R, int32_t G, int32_t rows,
                                  int32_t cluster_block_size, int32_t block_buckets, const int32_t* ends,
                                  int64_t row_tables, int64_t group_tables, int32_t* counts, void* stream) {
  LSA_REQUIRE(positions && counts, LSA_ERR_NULL, "lsa_visible_counts: positions/counts NULL");
  LSA_REQUIRE(R >= 0 && G >= 1 && rows >= 0, LSA_ERR_SHAPE, "lsa_visible_counts: bad sizes");
  LSA_REQUIRE(ends || (cluster_block_size >= 1 && block_buckets >= 0), LSA_ERR_SHAPE,
              "lsa_visible_counts: cluster_block_size must be >= 1");
  if (R * G == 0) return LSA_OK;
  const int64_t n = R * G;
  visible_counts_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(
      positions, R, G, rows, cluster_block_size, block_buckets, ends, row_tables, group_tables, counts);
  LSA_LAUNCHED("lsa_visible_counts");
  return LSA_OK;
}

extern "C" int lsa_score_rows(const void* queries, int q_dtype, int64_t R, int32_t G, int32_t D,
                              const void* centroids, int32_t N, int64_t row_tables, int64_t group_tables,
                              int score_mode, float* scores, void* stream) {
  LSA_REQUIRE(queries && centroids && scores, LSA_ERR_NULL, "lsa_score_rows: NULL pointer");
  LSA_TRY(check_dtype(q_dtype));
  LSA_TRY(check_dim(D));
  LSA_REQUIRE(score_mode == LSA_SCORE_BF16 || score_mode == LSA_SCORE_F32, LSA_ERR_DTYPE, "bad score mode");
  LSA_TRY(check_query_aligned(queries, q_dtype, D));
  LSA_REQUIRE(R >= 0 && G >= 1 && N >= 0 && R * G <= 0x7FFFFFFF, LSA_ERR_SHAPE, "lsa_score_rows: bad sizes");
  if (R * G == 0 || N == 0) return LSA_OK;
  LSA_REQUIRE((N + 15) / 16 <= 65535, LSA_ERR_SHAPE, "lsa_score_rows: %d columns exceed the grid", N);
  const dim3 grid((unsigned)(R * G), (unsigned)((N + 15) / 16));
  const bool bf16 = score_mode == LSA_SCORE_BF16;
  hipStream_t s = (hipStream_t)stream;
  LSA_DISPATCH_QT(q_dtype, LSA_DISPATCH_SPAN(D / 16, {
    if (bf16)
      score_rows_kernel<QT, bf16_t, SPAN><<<grid, LSA_BLOCK, 0, s>>>((const QT*)queries, G,
                                                                    (const bf16_t*)centroids, N, row_tables,
                                                                    group_tables, true, scores);
    else
      score_rows_kernel<QT, float, SPAN><<<grid, LSA_BLOCK, 0, s>>>((const QT*)queries, G, (const float*)centroids,
                                                                   N, row_tables, group_tables, false, scores);
  }))
  LSA_LAUNCHED("lsa_score_rows");
  return LSA_OK;
}

extern "C" int lsa_pack_listing(const float* scores, const int32_t* counts, int64_t R, int32_t N, int64_t* keys,
                                void* stream) {
  LSA_REQUIRE(scores && counts && keys, LSA_ERR_NULL, "lsa_pack_listing: NULL pointer");
  LSA_REQUIRE(R >= 0 && N >= 0, LSA_ERR_SHAPE, "lsa_pack_listing: bad sizes");
  const int64_t n = R * N;
  if (n == 0) return LSA_OK;
  pack_listing_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(scores, counts, R,
                                                                                               N, keys);
  LSA_LAUNCHED("lsa_pack_listing");
  return LSA_OK;
}

extern "C" int lsa_unpack_ids(const int64_t* keys, int64_t n, int32_t* ids, void* stream) {
  LSA_REQUIRE(keys && ids, LSA_ERR_NULL, "lsa_unpack_ids: NULL pointer");
  LSA_REQUIRE(n >= 0, LSA_ERR_SHAPE, "lsa_unpack_ids: bad size");
  if (n == 0) return LSA_OK;
  unpack_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(keys, n, ids);
  LSA_LAUNCHED("lsa_unpack_ids");
  return LSA_OK;
}

template <typename Src>
static int launch_topk(Src src, int64_t R, int32_t W, int32_t k, int32_t k_out, int64_t* out, hipStream_t s) {
  const int kp = next_pow2(k_out);
  const bool lds_row = W + kp <= kMaxLdsKeys;
  const size_t shmem = sizeof(uint64_t) * ((size_t)kp + (lds_row ? (size_t)W : 0));
  if (lds_row)
    topk_kernel<Src, true><<<dim3((unsigned)R), LSA_BLOCK, shmem, s>>>(src, W, k, kp, k_out, out);
  else
    topk_kernel<Src, false><<<dim3((unsigned)R), LSA_BLOCK, shmem, s>>>(src, W, k, kp, k_out, out);
  return LSA_OK;
}

extern "C" int lsa_topk_keys(const int64_t* keys, const int32_t* counts, int64_t R, int32_t W, int32_t k,
                             int64_t* out, void* stream) {
  LSA_REQUIRE(keys && out, LSA_ERR_NULL, "lsa_topk_keys: NULL pointer");
  LSA_REQUIRE(R >= 0 && W >= 1 && k >= 1 && k <= W, LSA_ERR_SHAPE, "lsa_topk_keys: need 1 <= k <= W (k=%d W=%d)", k,
              W);
  LSA_REQUIRE(k <= kMaxLdsKeys, LSA_ERR_SHAPE, "lsa_topk_keys: k=%d exceeds %d", k, kMaxLdsKeys);
  LSA_REQUIRE(R <= 0x7FFFFFFF, LSA_ERR_SHAPE, "lsa_topk_keys: too many rows");
  if (R == 0) return LSA_OK;
  launch_topk(KeySource{keys, counts, W}, R, W, k, k, out, (hipStream_t)stream);
  LSA_LAUNCHED("lsa_topk_keys");
  return LSA_OK;
}

extern "C" int lsa_select_topk_scores(const float* scores, const int32_t* lengths, int64_t R, int32_t N,
                                      int32_t top_p, int64_t* out, void* stream) {
  LSA_REQUIRE(scores && lengths && out, LSA_ERR_NULL, "lsa_select_topk_scores: NULL pointer");
  LSA_REQUIRE(R >= 0 && N >= 1 && top_p >= 1, LSA_ERR_SHAPE, "lsa_select_topk_scores: bad sizes");
  const int keep = top_p < N ? top_p : N;
  LSA_REQUIRE(next_pow2(keep) <= kMaxLdsKeys, LSA_ERR_SHAPE, "lsa_select_topk_scores: top_p %d too large", top_p);
  LSA_REQUIRE(R <= 0x7FFFFFFF, LSA_ERR_SHAPE, "lsa_select_topk_scores: too many rows");
  if (R == 0) return LSA_OK;
  launch_topk(ScoreSource{scores, lengths, N}, R, N, keep, next_pow2(keep), out, (hipStream_t)stream);
  LSA_LAUNCHED("lsa_select_topk_scores");
  return LSA_OK;
}

extern "C" int lsa_expand(const void* picks, int picks_are_keys, int64_t R, int32_t G, int32_t P,
                          const int32_t* members, int32_t rows, int32_t cap, int64_t row_tables, int64_t group_tables,
                          const int32_t* positions, const lsa_slot_map* slots, int32_t window, int32_t sink,
                          int32_t top_k, int32_t* lists, int32_t* lengths, void* stream) {
  LSA_REQUIRE(picks && members && positions && lists && lengths, LSA_ERR_NULL, "lsa_expand: NULL pointer");
  SlotMap sm;
  LSA_TRY(check_slots("lsa_expand", slots, &sm));
  LSA_TRY(check_tables(rows, cap, row_tables, group_tables));
  LSA_TRY(check_aligned(nullptr, 16, LSA_SCORE_BF16, members, cap));
  LSA_REQUIRE(R >= 0 && G >= 1 && P >= 0 && P <= 2 * kMaxLdsKeys, LSA_ERR_SHAPE, "lsa_expand: bad sizes (P=%d)", P);
  LSA_REQUIRE(window >= 0 && sink >= 0 && top_k >= 0, LSA_ERR_SHAPE, "lsa_expand: window/sink/top_k must be >= 0");
  LSA_REQUIRE(R * G <= 0x7FFFFFFF, LSA_ERR_SHAPE, "lsa_expand: too many rows");
  if (R * G == 0) return LSA_OK;
  const size_t shmem = sizeof(int32_t) * (size_t)(P > 0 ? P : 1);
  hipStream_t s = (hipStream_t)stream;
  if (picks_are_keys)
    expand_kernel<true><<<dim3((unsigned)(R * G)), LSA_BLOCK, shmem, s>>>(picks, G, P, members, rows, cap, row_tables,
                                                                        group_tables, positions, sm, window, sink,
                                                                        top_k, lists, lengths);
  else
    expand_kernel<false><<<dim3((unsigned)(R * G)), LSA_BLOCK, shmem, s>>>(picks, G, P, members, rows, cap,
                                                                         row_tables, group_tables, positions, sm,
                                                                         window, sink, top_k, lists, lengths);
  LSA_LAUNCHED("lsa_expand");
  return LSA_OK;
}

static int flat_picks(int32_t top_p, int32_t rows) { return top_p < rows ? top_p : rows; }

extern "C" size_t lsa_select_flat_scratch_bytes(int64_t R, int32_t G, int32_t top_p, int32_t N, int32_t splits) {
  (void)top_p;
  if (splits <= 1 || R <= 0 || G <= 0 || N <= 0) return 0;
  return (size_t)(R * G) * (size_t)N * sizeof(uint64_t);
}

extern "C" int lsa_select_flat(const void* queries, int q_dtype, int64_t R, int32_t G, int32_t D,
                               const void* centroids, const int32_t* members, const int32_t* ends,
                               int32_t table_flags, int32_t rows,
                               int32_t cap, int64_t row_tables, int64_t group_tables, int score_mode,
                               const int32_t* positions, const lsa_slot_map* slots, int32_t cluster_block_size,
                               int32_t block_buckets, int32_t top_p, int32_t window, int32_t sink, int32_t top_k,
                               int32_t splits, int32_t* counters, void* scratch, size_t scratch_bytes,
                               int32_t* lists, int32_t* lengths, void* stream) {
  LSA_REQUIRE(queries && centroids && members && positions && lists && lengths, LSA_ERR_NULL,
              "lsa_select_flat: NULL pointer");
  SlotMap sm;
  LSA_TRY(check_slots("lsa_select_flat", slots, &sm));
  LSA_TRY(check_dtype(q_dtype));
  LSA_TRY(check_dim(D));
  LSA_TRY(check_tables(rows, cap, row_tables, group_tables));
  LSA_REQUIRE(score_mode == LSA_SCORE_BF16 || score_mode == LSA_SCORE_F32, LSA_ERR_DTYPE, "bad score mode");
  LSA_TRY(check_aligned(centroids, D, score_mode, members, cap));
  LSA_TRY(check_query_aligned(queries, q_dtype, D));
  LSA_REQUIRE(R >= 0 && G >= 1 && R * G <= 0x7FFFFFFF, LSA_ERR_SHAPE, "lsa_select_flat: bad sizes");
  LSA_REQUIRE(top_p >= 1 && window >= 0 && sink >= 0 && top_k >= 0, LSA_ERR_SHAPE,
              "lsa_select_flat: top_p >= 1, window/sink/top_k >= 0");
  LSA_REQUIRE(ends || cluster_block_size >= 1, LSA_ERR_SHAPE, "lsa_select_flat: cluster_block_size must be >= 1");
  LSA_REQUIRE((table_flags & ~(LSA_TABLE_SPANS | LSA_TABLE_BLOCK_VISIBLE)) == 0, LSA_ERR_SHAPE,
              "lsa_select_flat: unknown table flags %d", table_flags);
  LSA_REQUIRE(ends || cluster_block_size >= 1 || !(table_flags & LSA_TABLE_BLOCK_VISIBLE), LSA_ERR_SHAPE,
              "lsa_select_flat: cluster_block_size must be >= 1");
  LSA_REQUIRE(!(table_flags & LSA_TABLE_SPANS) || ends, LSA_ERR_SHAPE,
              "lsa_select_flat: LSA_TABLE_SPANS needs the span ends");
  LSA_REQUIRE(splits >= 1 && splits <= 256 && splits <= rows, LSA_ERR_SHAPE,
              "lsa_select_flat: splits in [1, min(256, rows)], got %d", splits);
  const int K = flat_picks(top_p, rows);
  const int cs = (rows + splits - 1) / splits;
  const int kp = next_pow2(K);
  LSA_REQUIRE(rows + kp <= kMaxLdsKeys, LSA_ERR_SHAPE,
              "lsa_select_flat: %d columns + %d picks exceed %d LDS keys", rows, kp, kMaxLdsKeys);
  const size_t need = lsa_select_flat_scratch_bytes(R, G, top_p, rows, splits);
  LSA_REQUIRE(need == 0 || (scratch && counters && scratch_bytes >= need), LSA_ERR_WORKSPACE,
              "lsa_select_flat: counters/scratch missing or scratch %zu < %zu bytes", scratch_bytes, need);
  if (R * G == 0) return LSA_OK;
  FlatArgs a;
  a.R = R; a.G = G; a.rows = rows; a.cap = cap; a.row_tables = row_tables; a.group_tables = group_tables;
  a.centroids = centroids; a.members = members; a.ends = ends; a.positions = positions;
  a.vends = (table_flags & LSA_TABLE_BLOCK_VISIBLE) ? nullptr : ends;
  a.cluster_block = cluster_block_size; a.block_buckets = block_buckets;
  a.K = K; a.kp = kp; a.window = window; a.sink = sink; a.top_k = top_k;
  a.S = splits; a.cs = cs;
  a.ws_count = counters;
  a.ws_keys = need ? (uint64_t*)scratch : nullptr;
  a.slots = sm;
  a.lists = lists; a.lengths = lengths;
  a.spans = (table_flags & LSA_TABLE_SPANS) && K <= 16 * LSA_BLOCK ? 1 : 0;  // more picks: the member rows
  // the list row is staged in LDS when it fits beside the keys (coalesced row stores)
  const int width = top_k + window + sink;
  const size_t base_lds = sizeof(uint64_t) * (((size_t)rows + kp + 1) & ~(size_t)1);
  const size_t stage_lds = sizeof(int32_t) * ((size_t)width + 4);
  a.stage = (!a.spans && width % 4 == 0 && ((uintptr_t)lists % 16) == 0 && base_lds + stage_lds <= kMaxDynLds) ? 1 : 0;
  // span tables with more than 64 picks stage the row in the keys region, dead after the top-K
  a.wide_stage = (a.spans && K > LSA_WAVE && width % 4 == 0 && ((uintptr_t)lists % 16) == 0 &&
                  ((4 * (size_t)K + 15) & ~(size_t)15) + stage_lds <= sizeof(uint64_t) * (size_t)rows)
                     ? 1 : 0;
  a.screen = splits == 1 && score_mode == LSA_SCORE_BF16 && screen_pays(D, rows, K) ? 1 : 0;
  size_t shmem = base_lds + (a.stage ? stage_lds : 0);
  const size_t screen_lds = sizeof(ScreenLds) + sizeof(uint64_t) * (size_t)kp;
  if (a.screen && screen_lds > shmem) shmem = screen_lds;
  const dim3 grid((unsigned)(R * G), (unsigned)splits);
  const bool bf16 = score_mode == LSA_SCORE_BF16;
  hipStream_t s = (hipStream_t)stream;
  LSA_DISPATCH_QT(q_dtype, LSA_DISPATCH_SPAN(D / 16, {
    if (bf16) select_flat_kernel<QT, bf16_t, SPAN><<<grid, LSA_BLOCK, shmem, s>>>((const QT*)queries, true, a);
    else select_flat_kernel<QT, float, SPAN><<<grid, LSA_BLOCK, shmem, s>>>((const QT*)queries, false, a);
  }))
  LSA_LAUNCHED("lsa_select_flat");
  return LSA_OK;
}

extern "C" int lsa_select_tree(const void* queries, int q_dtype, int64_t R, int32_t G, int32_t D,
                               const void* node_centroids, const int32_t* children, int32_t n_nodes,
                               int32_t node_size, const void* centroids, const int32_t* members, const int32_t* ends,
                               int32_t table_flags, int32_t rows, int32_t cap, int64_t row_tables, int64_t group_tables, int score_mode,
                               const int32_t* positions, const lsa_slot_map* slots, int32_t cluster_block_size,
                               int32_t block_buckets, int32_t node_block, int32_t beam_width, int32_t top_p,
                               int32_t window, int32_t sink, int32_t top_k, int32_t* lists, int32_t* lengths,
                               void* stream) {
  LSA_REQUIRE(queries && node_centroids && children && centroids && members && positions && lists && lengths,
              LSA_ERR_NULL, "lsa_select_tree: NULL pointer");
  SlotMap sm;
  LSA_TRY(check_slots("lsa_select_tree", slots, &sm));
  LSA_TRY(check_dtype(q_dtype));
  LSA_TRY(check_dim(D));
  LSA_TRY(check_tables(rows, cap, row_tables, group_tables));
  LSA_REQUIRE(score_mode == LSA_SCORE_BF16 || score_mode == LSA_SCORE_F32, LSA_ERR_DTYPE, "bad score mode");
  LSA_TRY(check_aligned(centroids, D, score_mode, members, cap));
  LSA_TRY(check_aligned(node_centroids, D, score_mode, nullptr, cap));
  LSA_TRY(check_query_aligned(queries, q_dtype, D));
  LSA_REQUIRE(R >= 0 && G >= 1 && R * G <= 0x7FFFFFFF, LSA_ERR_SHAPE, "lsa_select_tree: bad sizes");
  LSA_REQUIRE(n_nodes >= 1 && node_size >= 1 && beam_width >= 1 && top_p >= 1 && node_block >= 1, LSA_ERR_SHAPE,
              "lsa_select_tree: n_nodes, node_size, node_block, beam_width, top_p >= 1");
  LSA_REQUIRE(window >= 0 && sink >= 0 && top_k >= 0, LSA_ERR_SHAPE, "lsa_select_tree: window/sink/top_k >= 0");
  LSA_REQUIRE(ends || cluster_block_size >= 1, LSA_ERR_SHAPE, "lsa_select_tree: cluster_block_size must be >= 1");
  LSA_REQUIRE((table_flags & ~(LSA_TABLE_SPANS | LSA_TABLE_BLOCK_VISIBLE)) == 0, LSA_ERR_SHAPE,
              "lsa_select_tree: unknown table flags %d", table_flags);
  LSA_REQUIRE(!(table_flags & LSA_TABLE_BLOCK_VISIBLE) || cluster_block_size >= 1, LSA_ERR_SHAPE,
              "lsa_select_tree: cluster_block_size must be >= 1");
  LSA_REQUIRE(!(table_flags & LSA_TABLE_SPANS) || ends, LSA_ERR_SHAPE,
              "lsa_select_tree: LSA_TABLE_SPANS needs the span ends");
  const int beam = beam_width < n_nodes ? beam_width : n_nodes;
  // fresh buckets [covered, visible): fewer than node_block past the made nodes, or every
  // bucket past the nodes' reach
  const int64_t reach = (int64_t)n_nodes * node_size;
  const int64_t max_fresh = rows - reach > (int64_t)node_block - 1 ? rows - reach : node_block - 1;
  const int64_t cand_cap = (int64_t)beam * node_size + (max_fresh < rows ? max_fresh : rows);
  LSA_REQUIRE(n_nodes <= kMaxLdsKeys && cand_cap <= kMaxLdsKeys && top_p <= kMaxLdsKeys, LSA_ERR_SHAPE,
              "lsa_select_tree: %d nodes / %lld candidates exceed %d", n_nodes, (long long)cand_cap, kMaxLdsKeys);
  if (R * G == 0) return LSA_OK;
  TreeArgs a;
  a.R = R; a.G = G; a.node_centroids = node_centroids; a.children = children; a.n_nodes = n_nodes;
  a.node_size = node_size; a.centroids = centroids; a.members = members; a.ends = ends; a.rows = rows; a.cap = cap;
  a.vends = (table_flags & LSA_TABLE_BLOCK_VISIBLE) ? nullptr : ends;
  a.row_tables = row_tables; a.group_tables = group_tables; a.positions = positions;
  a.cluster_block = cluster_block_size; a.block_buckets = block_buckets; a.node_block = node_block;
  a.beam = beam_width; a.top_p = top_p;
  a.nodes_pow2 = next_pow2(n_nodes); a.beam_pow2 = next_pow2(beam); a.cand_cap = (int)cand_cap;
  a.cand_pow2 = next_pow2((int)(cand_cap > 0 ? cand_cap : 1)); a.top_pow2 = next_pow2(top_p);
  a.window = window; a.sink = sink; a.top_k = top_k; a.lists = lists; a.lengths = lengths; a.slots = sm;
  a.spans = (table_flags & LSA_TABLE_SPANS) && top_p <= 16 * LSA_BLOCK ? 1 : 0;  // else the member rows
  a.screen1 = score_mode == LSA_SCORE_BF16 && screen_pays(D, n_nodes, beam) ? 1 : 0;
  a.screen0 = score_mode == LSA_SCORE_BF16 && screen_pays(D, a.cand_pow2, top_p < a.cand_pow2 ? top_p : a.cand_pow2)
                  ? 1 : 0;
  const int keys_slots = a.nodes_pow2 > a.cand_pow2 ? a.nodes_pow2 : a.cand_pow2;
  const int best_slots = a.beam_pow2 > a.top_pow2 ? a.beam_pow2 : a.top_pow2;
  const int cand_slots = a.cand_pow2 > top_p ? a.cand_pow2 : top_p;
  const size_t shmem = sizeof(uint64_t) * (size_t)(keys_slots + best_slots) + sizeof(int32_t) * (size_t)cand_slots;
  LSA_REQUIRE(shmem <= 8 * (size_t)kMaxLdsKeys, LSA_ERR_SHAPE, "lsa_select_tree: %zu bytes of LDS needed", shmem);
  const bool bf16 = score_mode == LSA_SCORE_BF16;
  hipStream_t s = (hipStream_t)stream;
  LSA_DISPATCH_QT(q_dtype, LSA_DISPATCH_SPAN(D / 16, {
    if (bf16) select_tree_kernel<QT, bf16_t, SPAN><<<dim3((unsigned)(R * G)), LSA_BLOCK, shmem, s>>>((const QT*)queries,
                                                                                                   true, a);
    else select_tree_kernel<QT, float, SPAN><<<dim3((unsigned)(R * G)), LSA_BLOCK, shmem, s>>>((const QT*)queries,
                                                                                             false, a);
  }))
  LSA_LAUNCHED("lsa_select_tree");
  return LSA_OK;
}

extern "C" int lsa_index_queries(const void* q, int q_dtype, int64_t B, int64_t T, int32_t Hq, int32_t Hkv, int32_t D,
                                 int32_t chunk, float* out, void* stream) {
  LSA_REQUIRE(q && out, LSA_ERR_NULL, "lsa_index_queries: NULL pointer");
  LSA_TRY(check_dtype(q_dtype));
  LSA_REQUIRE(B >= 0 && T >= 0 && Hq >= 1 && Hkv >= 1 && D >= 1 && chunk >= 1, LSA_ERR_SHAPE,
              "lsa_index_queries: bad sizes");
  LSA_REQUIRE(Hq % Hkv == 0, LSA_ERR_SHAPE, "lsa_index_queries: Hq %d not a multiple of Hkv %d", Hq, Hkv);
  const int64_t n = B * (T / chunk) * Hkv * D;
  if (n == 0) return LSA_OK;
  hipStream_t s = (hipStream_t)stream;
  const int esize = q_dtype == LSA_F32 ? 4 : 2;
  const bool vec = D % 4 == 0 && ((uintptr_t)q % (4 * esize)) == 0;  // 4 dims a thread
  const dim3 grid((unsigned)((n / (vec ? 4 : 1) + 255) / 256));
  if (vec) {
    LSA_DISPATCH_QT(q_dtype,
                    { index_queries_kernel<QT, 4><<<grid, 256, 0, s>>>((const QT*)q, B, T, Hq, Hkv, D, chunk, out); })
  } else {
    LSA_DISPATCH_QT(q_dtype,
                    { index_queries_kernel<QT, 1><<<grid, 256, 0, s>>>((const QT*)q, B, T, Hq, Hkv, D, chunk, out); })
  }
  LSA_LAUNCHED("lsa_index_queries");
  return LSA_OK;
}

extern "C" int lsa_bucket_centroids(const void* keys, int k_dtype, int64_t tokens, int64_t token_stride,
                                    int64_t batch_stride,
                                    int32_t kv_heads, int32_t D, const int32_t* members, int64_t n_tables,
                                    int32_t rows, int32_t cap, int centroid_mode, float* out_f32, uint16_t* out_bf16,
                                    void* stream) {
  LSA_REQUIRE(keys && members && out_f32, LSA_ERR_NULL, "lsa_bucket_centroids: NULL pointer");
  LSA_TRY(check_dtype(k_dtype));
  LSA_REQUIRE(D >= 1 && D <= 512 && kv_heads >= 1 && n_tables >= 0 && rows >= 0 && cap >= 1 && tokens >= 0,
              LSA_ERR_SHAPE,
              "lsa_bucket_centroids: bad sizes");
  LSA_REQUIRE(centroid_mode == LSA_CENTROID_MEAN || centroid_mode == LSA_CENTROID_NORMALIZED ||
                  centroid_mode == LSA_CENTROID_SUM,
              LSA_ERR_SHAPE,
              "lsa_bucket_centroids: bad centroid mode");
  const int64_t n = n_tables * rows;
  if (n == 0) return LSA_OK;
  LSA_REQUIRE(n <= 0x7FFFFFFF, LSA_ERR_SHAPE, "lsa_bucket_centroids: too many buckets");
  hipStream_t s = (hipStream_t)stream;
  LSA_DISPATCH_QT(k_dtype, {
    centroids_kernel<QT><<<dim3((unsigned)n), LSA_BLOCK, 0, s>>>((const QT*)keys, tokens, token_stride, batch_stride,
                                                                kv_heads,
                                                                D, members, rows, cap, centroid_mode, out_f32,
                                                                out_bf16);
  })
  LSA_LAUNCHED("lsa_bucket_centroids");
  return LSA_OK;
}
