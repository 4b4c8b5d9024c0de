// Device side of the fused decode step: arguments, LDS layouts, the select and reader
// roles and the kernel, plus the per-element-type launcher that each decode_<type>.hip
// instantiates (one translation unit per type, compiled in parallel).
#pragma once

#include <math.h>

#include "lsa_abi_common.h"
#include "lsa_read_dev.h"
#include "lsa_screen_dev.h"
#include "lsa_select_dev.h"

namespace lsa {
namespace decode {

constexpr int kMaxPicks = LSA_WAVE;  // the record of a unit is polled by one wave
constexpr int kMaxReaders = 256;     // readers per unit (split partials of the combine)
constexpr int kRecordCopies = 8;     // copies of every record, polled by different readers
constexpr size_t kMaxLds = 64 * 1024;
// Rank form (readers rank the select splits' published keys themselves): at most this many
// bucket rows a table (a reader holds their keys and span ends in LDS, a polling lane
// kRankKeysPerLane keys) and this many published key slots in all (they sit in the
// counters region, which must start zero).
constexpr int kRankMaxRows = 1024;
constexpr int kRankKeysPerLane = kRankMaxRows / LSA_WAVE;
constexpr int64_t kRankMaxSlots = 1 << 16;

// Phase hooks: no-ops unless a build defines DECODE_MARK(k) (timestamps for profiling; k < 16:
// 0-6 the select and reader phases, 7 a ranking reader holding its picks, 8-11 the
// replicated select's).
#ifndef DECODE_MARK
#define DECODE_MARK(k) ((void)0)
#define DECODE_TRACE_BEGIN() ((void)0)
#define DECODE_TRACE_END() ((void)0)
#endif

struct DecodeArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  int64_t R;
  int G, Hq;
  int64_t Tk, kv_sb, kv_st, kv_sh;
  const void* centroids;
  const int32_t* members;
  const int32_t* ends;
  int rows, cap;
  int vec_rows;        // cap % 4 == 0 and the member table 16-byte aligned
  int spans;           // bucket row j holds exactly ids ends[j - 1] .. ends[j] - 1 (ends[-1] = 0)
  const int32_t* vends;  // the ends that decide visibility (nullptr: the closed-block rule)
  int64_t row_tables, group_tables;
  const int32_t* positions;
  int cluster_block, block_buckets;
  int K, kp, window, sink, top_k, W;
  int S, cs;           // select splits and columns per split
  int screen;          // S == 1 with bf16 tables that fit screen_topk: the select screens its table
  int span, NR;        // slots per read part, readers per unit
  int chunk;           // tiles of a reader's id chunk (the LDS holds chunk * span ids)
  // tree select (one workgroup a unit): node level over the bucket table
  int tree;                     // 1: the select role walks a one-level node tree
  const void* node_centroids;   // [tables, n_nodes, D], the centroid type
  const int32_t* children;      // [tables, n_nodes, node_size] bucket rows
  int n_nodes, node_size, node_block, beam;
  int ends4;                    // span ends readable as 16-byte vectors (rows % 4 == 0, aligned)
  int stash;                    // the tree select stages the children table and span ends in LDS
  int kids4;                    // the children table readable as 16-byte vectors
  int nodes_pow2, beam_pow2, cand_pow2, top_pow2;
  float scale_log2;
  int spin_limit;
  int skip_publish;    // test hook: select workgroups never publish (readers give up)
  int rank;            // rank form: splits publish their keys, every reader ranks them itself
  uint64_t* pub;       // rank form: [units][rows] published keys + 1 (0: not yet written)
  int* sel_count;      // [units] select arrivals
  int* rd_count;       // [units] reader arrivals
  int32_t* record;     // kRecordCopies copies, `cstride` words apart: [units][2K] words A then B
  int64_t cstride;
  uint64_t* ws_keys;   // [units][rows] (S > 1)
  float* ws_part;      // [units][NR][GQ*(D+2)] (NR > 1)
  int32_t* lists;      // [units][W]
  int32_t* lengths;    // [units]
  int32_t* status;     // optional: set to 1 by a reader whose wait timed out (system scope:
                       // the word may live in pinned host memory)
  SlotMap slots;       // a paged cache's slot table (table == nullptr: ids are cache rows)
};

struct SelLds {
  RadixState st;
  TopkScratch tks;
  int pick[kMaxPicks];
  int cnt[kMaxPicks];
  int first[kMaxPicks];  // span tables: the first kept id of each pick
  int rec[2 * kMaxPicks];
  int flag;
};

template <int D, int GQ>
struct RdLds {
  ReadLds<D, GQ, kMaxReaders> rd;
  int pick[kMaxPicks], start[kMaxPicks], n[kMaxPicks];
  int wcnt[LSA_WAVES];
  int filled, bad;
};

constexpr size_t sel_keys_offset() { return (sizeof(SelLds) + 15) & ~(size_t)15; }

// The tree select's LDS after its keys, picks, candidates and dedup bitmap (laid out in
// tree_role): where the stashed children table and span ends start, 16-byte aligned.
__host__ __device__ inline size_t tree_stash_offset(int nodes_pow2, int cand_pow2, int beam_pow2, int top_pow2,
                                                    int rows) {
  const size_t keys = (size_t)(nodes_pow2 > cand_pow2 ? nodes_pow2 : cand_pow2);
  const size_t best = (size_t)(beam_pow2 > top_pow2 ? beam_pow2 : top_pow2);
  const size_t end = sel_keys_offset() + sizeof(uint64_t) * (keys + best) + sizeof(int32_t) * (size_t)cand_pow2 +
                     sizeof(uint32_t) * (size_t)((rows + 31) / 32);
  return (end + 15) & ~(size_t)15;
}
// Bytes of the stash: the children table and the span ends, each rounded to 16 bytes.
__host__ __device__ inline size_t tree_stash_bytes(int words, int rows) {
  return sizeof(int32_t) * (size_t)(((words + 3) & ~3) + ((rows + 3) & ~3));
}
template <int D, int GQ>
constexpr size_t rd_ids_offset() {
  return (sizeof(RdLds<D, GQ>) + 15) & ~(size_t)15;
}

// A ranking reader's selection state, in the space of its id chunk (dead until the read):
// the top-K scratch, then the table's span ends [rows], then the keys [rows].
struct RankLds {
  RadixState st;
  TopkScratch tks;
  uint64_t best[kMaxPicks];
  int fast;  // wave 0 ranked the keys itself (wave_topk_hist)
};
template <int D, int GQ>
constexpr size_t rank_ends_offset() {
  return (rd_ids_offset<D, GQ>() + sizeof(RankLds) + 15) & ~(size_t)15;
}
template <int D, int GQ>
__host__ __device__ constexpr size_t rank_keys_offset(int rows) {
  return (rank_ends_offset<D, GQ>() + sizeof(int32_t) * (size_t)rows + 15) & ~(size_t)15;
}
template <int D, int GQ>
__host__ __device__ constexpr size_t rank_lds(int rows) {
  return rank_keys_offset<D, GQ>(rows) + sizeof(uint64_t) * (size_t)rows;
}

// The unit's index query slice of lane group p: fp32 mean of the group's GQ query rows
// (head order), rounded like load_query_slice in bf16 scoring.
template <typename QT, int SPAN, int GQ>
__device__ __forceinline__ void group_mean_slice(const QT* q, int p, bool bf16_mode, float* out) {
  constexpr int D = 16 * SPAN;
  SpanRaw<QT, SPAN> raw[GQ];
#pragma unroll
  for (int h = 0; h < GQ; ++h) raw[h].load(q + (int64_t)h * D + p * SPAN);
#pragma unroll
  for (int j = 0; j < SPAN; ++j) {
    float acc = 0.0f;
#pragma unroll
    for (int h = 0; h < GQ; ++h) acc += raw[h].at(j);
    const float x = acc / (float)GQ;
    out[j] = bf16_mode ? bf16_round(x) : x;
  }
}

__device__ __forceinline__ int64_t window_start_of(int64_t position, int window) {
  const int64_t ws = position + 1 - window;
  return ws > 0 ? ws : 0;
}

// Kept members (sink <= id < window start) of picks pick[0..K) (bucket rows of the member
// table `tab`, -1 = none) into cnt_out[0..K): wave w counts picks w, w + 4, ... eight at a
// time; a member row streams through the wave in 16-byte lane loads (256 slots per wave
// load; 64 four-byte loads without vec_rows), counted with ballots. Every thread calls it;
// cnt_out is complete after the caller's next barrier.
__device__ __forceinline__ void count_members(const DecodeArgs& a, const int32_t* tab, const int* pick, int* cnt_out,
                                              int64_t wstart) {
  const int lane = threadIdx.x & (LSA_WAVE - 1), w = threadIdx.x / LSA_WAVE;
  constexpr int MJ = 8;
  for (int jb = 0; jb < a.K; jb += MJ * LSA_WAVES) {
    int cnt[MJ];
    int b[MJ];
#pragma unroll
    for (int m = 0; m < MJ; ++m) {
      const int j = jb + m * LSA_WAVES + w;
      b[m] = j < a.K ? pick[j] : -1;
      cnt[m] = 0;
    }
    const int step = a.vec_rows ? 4 * LSA_WAVE : LSA_WAVE;
    for (int c0 = 0; c0 < a.cap; c0 += step) {
      if (a.vec_rows) {
        int4 x[MJ];
        const int e = c0 + 4 * lane;
#pragma unroll
        for (int m = 0; m < MJ; ++m) {  // unconditional (clamped) loads: all in flight
          const bool ok = b[m] >= 0 && e < a.cap;
          x[m] = *(const int4*)(tab + (ok ? (int64_t)b[m] * a.cap + e : 0));
          if (!ok) x[m] = make_int4(-1, -1, -1, -1);
        }
#pragma unroll
        for (int m = 0; m < MJ; ++m) {
          const int32_t v4[4] = {x[m].x, x[m].y, x[m].z, x[m].w};
#pragma unroll
          for (int k = 0; k < 4; ++k)
            cnt[m] += (int)__popcll(__ballot(v4[k] >= a.sink && (int64_t)v4[k] < wstart));
        }
      } else {
        int32_t x[MJ];
        const int e = c0 + lane;
#pragma unroll
        for (int m = 0; m < MJ; ++m) {
          const bool ok = b[m] >= 0 && e < a.cap;
          x[m] = tab[ok ? (int64_t)b[m] * a.cap + e : 0];
          if (!ok) x[m] = -1;
        }
#pragma unroll
        for (int m = 0; m < MJ; ++m) cnt[m] += (int)__popcll(__ballot(x[m] >= a.sink && (int64_t)x[m] < wstart));
      }
    }
    if (lane == 0) {
#pragma unroll
      for (int m = 0; m < MJ; ++m) {
        const int j = jb + m * LSA_WAVES + w;
        if (j < a.K) cnt_out[j] = cnt[m];
      }
    }
  }
}

// The select's last step, once sh.pick[0..K) holds the unit's picks (bucket rows, -1 =
// none): each pick's kept members are counted, the list length written and the unit's
// record published (every copy, write-through). Every thread calls it.
__device__ __forceinline__ void publish_picks(const DecodeArgs& a, SelLds& sh, int64_t i, int64_t t, int64_t position,
                                              const int32_t* ends) {
  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1), w = tid / LSA_WAVE;
  // kept members of every pick (sink <= id < window start). Span tables: the range
  // [ends[b - 1], ends[b]) clipped to [sink, window start), from two ends words. Otherwise
  // counted from the member rows (count_members)
  const int32_t* tab = a.members + t * (int64_t)a.rows * a.cap;
  const int64_t wstart = window_start_of(position, a.window);
  if (a.spans) {
    if (w == 0 && lane < a.K) {
      const int b = sh.pick[lane];
      const int64_t begin = b > 0 ? ends[b - 1] : 0, end = b >= 0 ? ends[b] : 0;
      const int64_t lo = begin > a.sink ? begin : a.sink, hi = end < wstart ? end : wstart;
      sh.cnt[lane] = b >= 0 && hi > lo ? (int)(hi - lo) : 0;
      sh.first[lane] = (int)lo;
    }
  } else {
    count_members(a, tab, sh.pick, sh.cnt, wstart);
  }
  __syncthreads();
  DECODE_MARK(5);
  if (w == 0) {
    const int c = lane < a.K ? sh.cnt[lane] : 0;
    const int incl = wave_inclusive_sum(c);
    const int end = incl < a.top_k ? incl : a.top_k;
    if (lane < a.K) {
      sh.rec[lane] = (a.spans ? sh.first[lane] : sh.pick[lane]) + 2;  // pick, or its first kept id
      sh.rec[a.K + lane] = end + 1;
    }
    if (lane == a.K - 1) {
      const int64_t n_win = position + 1 - wstart > 0 ? position + 1 - wstart : 0;
      const int64_t n_sink = a.sink < wstart ? a.sink : wstart;
      a.lengths[i] = end + (int)n_win + (int)n_sink;
    }
  }
  __syncthreads();
  if (a.skip_publish) return;
  // every copy of the record, write-through
  const int words = 2 * a.K;
  for (int x = tid; x < kRecordCopies * words; x += LSA_BLOCK) {
    const int c = x / words, k = x - c * words;
    coherent_store_i32(a.record + c * a.cstride + i * words + k, sh.rec[k]);
  }
  DECODE_MARK(6);
}

template <typename T, typename CT, int D, int GQ>
__device__ __forceinline__ void select_role(const DecodeArgs& a, char* smem, int64_t i, int s) {
  constexpr int SPAN = D / 16;
  constexpr bool BF16_MODE = __is_same(CT, bf16_t);
  SelLds& sh = *(SelLds*)smem;
  uint64_t* keys = (uint64_t*)(smem + sel_keys_offset());  // [rows]
  uint64_t* best = keys + a.rows;                           // [kp]
  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1), w = tid / LSA_WAVE;
  const int64_t r = (uint32_t)i / (uint32_t)a.G;  // units < 2^31 (checked on the host): 32-bit division
  const int g = (int)((uint32_t)i % (uint32_t)a.G);
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
  DECODE_MARK(0);

  float qs[SPAN];
  const T* qrow = (const T*)a.q + (r * a.Hq + (int64_t)g * GQ) * D;
  constexpr int GROUPS = LSA_BLOCK / 16;
  bool picked = false;
  if constexpr (__is_same(CT, bf16_t) && D >= 32 && D <= 128) {
    if (a.screen) {  // one split scores the whole table: on the matrix cores, exact (screen_topk)
      group_mean_slice<T, SPAN, GQ>(qrow, tid & 15, true, qs);
      ScreenLds& scr = *(ScreenLds*)(smem + sel_keys_offset());  // in place of the keys
      uint64_t* sbest = (uint64_t*)(smem + sel_keys_offset() + sizeof(ScreenLds));
      // span ends are nondecreasing: the visible rows are a prefix, counted once (a span-end
      // load per screened row would sit on the screen's critical path)
      __shared__ int vis_lds[2 * LSA_WAVES];
      const int nvis = vends ? visible_count_block(position, a.rows, vends, vis_lds) : vis;
      screen_topk<D, 4>(
          qs, cent, a.rows, [](int j) { return j; }, [&](int j) { return j < nvis; }, a.K, a.kp, sbest, scr);
      for (int j = tid; j < a.K; j += LSA_BLOCK) {
        const int32_t b = key_column(u_to_key(sbest[j]));
        sh.pick[j] = (b >= 0 && b < a.rows) ? b : -1;
      }
      __syncthreads();
      picked = true;
    }
  }
  if (picked) {
    DECODE_MARK(4);
  } else if (n_local <= 2 * GROUPS) {
    // one memory round trip: the group's query rows, the (at most) two centroid rows each
    // 16-lane group scores and their span ends are all in flight before the index query
    // is formed (group_mean_slice's arithmetic) and the rows are scored (score_keys')
    const int grp = tid >> 4, p = tid & 15;
    SpanRaw<T, SPAN> qraw[GQ];
#pragma unroll
    for (int h = 0; h < GQ; ++h) qraw[h].load(qrow + (int64_t)h * D + p * SPAN);
    SpanRaw<CT, SPAN> craw[2];
    int col[2];
    int32_t e[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int j = k * GROUPS + grp;
      col[k] = j < n_local ? c0 + j : -1;
      const int cc = col[k] >= 0 ? col[k] : 0;  // row 0: a split may hold no column (c0 >= rows)
      craw[k].load(cent + (int64_t)cc * D + p * SPAN);
      e[k] = vends ? vends[cc] : 0;
    }
#pragma unroll
    for (int j = 0; j < SPAN; ++j) {
      float acc = 0.0f;
#pragma unroll
      for (int h = 0; h < GQ; ++h) acc += qraw[h].at(j);
      const float x = acc / (float)GQ;
      qs[j] = BF16_MODE ? bf16_round(x) : x;
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      double acc = 0.0;
#pragma unroll
      for (int x = 0; x < SPAN; ++x) acc = fma((double)qs[x], (double)craw[k].at(x), acc);
      const float sc = score_tree16(acc);
      const bool keep = col[k] >= 0 && (vends ? (int64_t)e[k] <= lim : col[k] < vis);
      if (p == 0 && col[k] >= 0) keys[col[k]] = keep ? key_to_u(pack_key(sc, col[k])) : 0;
    }
  } else {
    group_mean_slice<T, SPAN, GQ>(qrow, tid & 15, BF16_MODE, qs);
    score_keys<CT, SPAN>(
        qs, cent, D, n_local, [&](int j) { return c0 + j; },
        [&](int j) { return vends ? (int64_t)vends[c0 + j] <= lim : c0 + j < vis; }, keys + c0);
  }
  if (!picked) {
    DECODE_MARK(1);

    if (a.rank) {  // publish the keys (+ 1, so that a written slot is nonzero); the readers rank them
      __syncthreads();
      if (a.skip_publish) return;
      uint64_t* mine = a.pub + i * (int64_t)a.rows;
      for (int j = tid; j < n_local; j += LSA_BLOCK) coherent_store_u64(mine + c0 + j, keys[c0 + j] + 1);
      DECODE_MARK(6);
      return;
    }
    if (a.S > 1) {
      __syncthreads();
      uint64_t* mine = a.ws_keys + i * (int64_t)a.rows;
      for (int j = tid; j < n_local; j += LSA_BLOCK) coherent_store_u64(mine + c0 + j, keys[c0 + j]);
      if (!arrive_last(&a.sel_count[i], a.S, &sh.flag)) return;
      DECODE_MARK(2);
      for (int jb = 0; jb < a.rows; jb += 4 * LSA_BLOCK) {
        uint64_t x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int j = jb + u * LSA_BLOCK + tid;
          x[u] = coherent_load_u64(mine + (j < a.rows ? j : 0));
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int j = jb + u * LSA_BLOCK + tid;
          if (j < a.rows) keys[j] = x[u];
        }
      }
    }
    __syncthreads();
    DECODE_MARK(3);
    block_topk_sorted(keys, a.rows, a.K, a.kp, best, &sh.tks, &sh.st);
    for (int j = tid; j < a.K; j += LSA_BLOCK) {
      const int32_t b = key_column(u_to_key(best[j]));
      sh.pick[j] = (b >= 0 && b < a.rows) ? b : -1;
    }
    __syncthreads();
    DECODE_MARK(4);
  }

  publish_picks(a, sh, i, t, position, ends);
}

// The tree select of unit i (one workgroup; reference _tree.py:318-373 with one node
// level, the growth of :100-142 at page end V = the unit's visible bucket count): the
// made nodes are [0, C / node_size) with C = min(floor(V / node_block) * node_block,
// n_nodes * node_size); the best `beam` made nodes (a tie to the lower node), then the
// best top_p of their visible children plus the fresh buckets [C, V), each bucket once (an
// LDS bitmap over bucket ids), a tie to the lower bucket; exact canonical scores at both
// levels. The picks then go out as the flat select's do (publish_picks). The same
// selection as select_tree_kernel.
//
// Laid out for few memory round trips: the query rows, the first tree_node_rows() node
// rows of each 16-lane group and the span ends (16-byte loads, kTreeEndVecs a thread) are
// all in flight before any of them is used; the fresh buckets' rows (when at most
// kTreeFreshRows a group) are loaded while the beam is chosen. What remains on the chain:
// nodes -> beam -> children -> their rows -> picks.
constexpr int kTreeEndVecs = 2;       // 4-end vectors a thread counts from the first round trip
constexpr int kTreeFreshRows = 4;     // fresh bucket rows a 16-lane group loads ahead of the beam

template <typename CT>
constexpr int tree_node_rows() {  // node rows a 16-lane group loads in the first round trip
  return sizeof(CT) == 2 ? 8 : 4;
}

template <typename T, typename CT, int D, int GQ>
__device__ __forceinline__ void tree_role(const DecodeArgs& a, char* smem, int64_t i) {
  constexpr int SPAN = D / 16;
  constexpr int GROUPS = LSA_BLOCK / 16;
  constexpr int NB = tree_node_rows<CT>();
  constexpr bool BF16_MODE = __is_same(CT, bf16_t);
  SelLds& sh = *(SelLds*)smem;
  uint64_t* keys = (uint64_t*)(smem + sel_keys_offset());                 // [max(nodes_pow2, cand_pow2)]
  uint64_t* best = keys + max(a.nodes_pow2, a.cand_pow2);                 // [max(beam_pow2, top_pow2)]
  int32_t* cand = (int32_t*)(best + max(a.beam_pow2, a.top_pow2));        // [cand_pow2]
  uint32_t* seen = (uint32_t*)(cand + a.cand_pow2);                       // [(rows + 31) / 32]
  int32_t* kids_l = (int32_t*)(smem + tree_stash_offset(a.nodes_pow2, a.cand_pow2, a.beam_pow2, a.top_pow2,
                                                        a.rows));               // stash: [words] children
  int32_t* ends_l = kids_l + ((a.n_nodes * a.node_size + 3) & ~3);         // stash: [rows] span ends
  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1), w = tid / LSA_WAVE;
  const int grp = tid >> 4, p = tid & 15;
  const int64_t r = (uint32_t)i / (uint32_t)a.G;
  const int g = (int)((uint32_t)i % (uint32_t)a.G);
  const int64_t position = a.positions[r];
  const int64_t lim = position + 1;
  const int64_t t = r * a.row_tables + g * a.group_tables;
  const int32_t* ends = a.ends ? a.ends + t * a.rows : nullptr;
  const int n_nodes = a.n_nodes, ns = a.node_size, words = n_nodes * ns;
  const CT* ncent = (const CT*)a.node_centroids + t * (int64_t)n_nodes * D;
  const CT* bcent = (const CT*)a.centroids + t * (int64_t)a.rows * D;
  const int32_t* kids = a.children + t * (int64_t)words;
  const T* qrow = (const T*)a.q + (r * a.Hq + (int64_t)g * GQ) * D;
  DECODE_MARK(0);

  // round trip 1: query rows, node rows, span ends, children - all issued before any use
  SpanRaw<T, SPAN> qraw[GQ];
#pragma unroll
  for (int h = 0; h < GQ; ++h) qraw[h].load(qrow + (int64_t)h * D + p * SPAN);
  SpanRaw<CT, SPAN> nraw[NB];
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    const int j = k * GROUPS + grp;
    nraw[k].load(ncent + (int64_t)(j < n_nodes ? j : 0) * D + p * SPAN);
  }
  // span ends as 16-byte vectors when the table's rows allow (ends4), else one at a time
  const bool ends4 = ends && a.ends4;
  const int nvec = ends4 ? a.rows / 4 : 0;
  int4 ev[kTreeEndVecs];
#pragma unroll
  for (int m = 0; m < kTreeEndVecs; ++m) {
    const int x = tid + m * LSA_BLOCK;
    ev[m] = x < nvec ? ((const int4*)ends)[x] : make_int4(0x7FFFFFFF, 0x7FFFFFFF, 0x7FFFFFFF, 0x7FFFFFFF);
  }
  // the children table, for the LDS stash (the kept nodes' children then cost no round trip)
  const int nkv = a.stash && a.kids4 ? words / 4 : 0;
  int4 kv[kTreeEndVecs];
#pragma unroll
  for (int m = 0; m < kTreeEndVecs; ++m) {
    const int x = tid + m * LSA_BLOCK;
    kv[m] = nkv > 0 ? ((const int4*)kids)[x < nkv ? x : 0] : make_int4(-1, -1, -1, -1);
  }

  // the index query (group mean, rounded like the unfused select's), the node scores
  float qs[SPAN];
#pragma unroll
  for (int j = 0; j < SPAN; ++j) {
    float acc = 0.0f;
#pragma unroll
    for (int h = 0; h < GQ; ++h) acc += qraw[h].at(j);
    const float x = acc / (float)GQ;
    qs[j] = BF16_MODE ? bf16_round(x) : x;
  }
  float nsc[NB];
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    double acc = 0.0;
#pragma unroll
    for (int e = 0; e < SPAN; ++e) acc = fma((double)qs[e], (double)nraw[k].at(e), acc);
    nsc[k] = score_tree16(acc);
  }
  // visible buckets: span ends <= position + 1 (nondecreasing, so a count), or closed form
  int nv = 0;
  if (ends4) {
#pragma unroll
    for (int m = 0; m < kTreeEndVecs; ++m) {
      nv += ((int64_t)ev[m].x <= lim ? 1 : 0) + ((int64_t)ev[m].y <= lim ? 1 : 0);
      nv += ((int64_t)ev[m].z <= lim ? 1 : 0) + ((int64_t)ev[m].w <= lim ? 1 : 0);
      const int x = tid + m * LSA_BLOCK;
      if (a.stash && x < nvec) ((int4*)ends_l)[x] = ev[m];
    }
    for (int x = tid + kTreeEndVecs * LSA_BLOCK; x < nvec; x += LSA_BLOCK) {
      const int4 e = ((const int4*)ends)[x];
      nv += ((int64_t)e.x <= lim ? 1 : 0) + ((int64_t)e.y <= lim ? 1 : 0);
      nv += ((int64_t)e.z <= lim ? 1 : 0) + ((int64_t)e.w <= lim ? 1 : 0);
      if (a.stash) ((int4*)ends_l)[x] = e;
    }
  } else if (ends) {
    for (int x = tid; x < a.rows; x += LSA_BLOCK) {
      const int32_t e = ends[x];
      nv += (int64_t)e <= lim ? 1 : 0;
      if (a.stash) ends_l[x] = e;
    }
  }
  if (a.stash) {
#pragma unroll
    for (int m = 0; m < kTreeEndVecs; ++m) {
      const int x = tid + m * LSA_BLOCK;
      if (x < nkv) ((int4*)kids_l)[x] = kv[m];
    }
    for (int x = tid + kTreeEndVecs * LSA_BLOCK; x < nkv; x += LSA_BLOCK) ((int4*)kids_l)[x] = ((const int4*)kids)[x];
    if (!a.kids4) {
      for (int x = tid; x < words; x += LSA_BLOCK) kids_l[x] = kids[x];
    }
  }
  nv = wave_sum(nv);
  __shared__ int vis_lds[LSA_WAVES];
  if (lane == 0) vis_lds[w] = nv;
  for (int x = tid; x < (a.rows + 31) / 32; x += LSA_BLOCK) seen[x] = 0;
  __syncthreads();
  const int visible =
      max(0, a.vends ? vis_lds[0] + vis_lds[1] + vis_lds[2] + vis_lds[3]
                     : visible_count(position, a.rows, a.cluster_block, a.block_buckets, nullptr));
  const int covered = min(visible / a.node_block * a.node_block, n_nodes * ns);
  const int made = covered / ns;
  const int n_fresh = max(0, visible - covered);

  // the node keys (made nodes only); nodes past the first batch take another round trip
  if (p == 0) {
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int j = k * GROUPS + grp;
      if (j < n_nodes) keys[j] = j < made ? key_to_u(pack_key(nsc[k], j)) : 0;
    }
  }
  if (n_nodes > NB * GROUPS) score_slice_keys<CT, SPAN>(qs, ncent, D, NB * GROUPS, n_nodes, made, keys + NB * GROUPS);
  // the fresh buckets' rows, in flight while the beam is chosen
  const bool fresh_ahead = n_fresh <= kTreeFreshRows * GROUPS;
  SpanRaw<CT, SPAN> fraw[kTreeFreshRows];
  if (fresh_ahead) {
#pragma unroll
    for (int k = 0; k < kTreeFreshRows; ++k) {
      const int j = k * GROUPS + grp;
      fraw[k].load(bcent + (int64_t)(j < n_fresh ? covered + j : 0) * D + p * SPAN);
    }
  }
  __syncthreads();
  const int beam = min(a.beam, n_nodes);
  block_topk_sorted(keys, n_nodes, beam, a.beam_pow2, best, &sh.tks, &sh.st);
  DECODE_MARK(1);

  // candidates: the fresh buckets [covered, visible) (distinct; marked in the bitmap first),
  // then the kept nodes' visible children that are not already candidates
  const int n_kids = beam * ns;
  const int n_cand = n_fresh + n_kids;
  for (int j = tid; j < n_fresh; j += LSA_BLOCK) {
    const int c = covered + j;
    cand[j] = c;
    atomicOr(&seen[c >> 5], 1u << (c & 31));
  }
  if (fresh_ahead) {
#pragma unroll
    for (int k = 0; k < kTreeFreshRows; ++k) {
      const int j = k * GROUPS + grp;
      double acc = 0.0;
#pragma unroll
      for (int e = 0; e < SPAN; ++e) acc = fma((double)qs[e], (double)fraw[k].at(e), acc);
      const float sc = score_tree16(acc);
      if (p == 0 && j < n_fresh) keys[j] = key_to_u(pack_key(sc, covered + j));
    }
  }
  __syncthreads();  // the fresh buckets' bits
  for (int m = tid; m < n_kids; m += LSA_BLOCK) {
    const int node = key_column(u_to_key(best[m / ns]));
    int32_t c = -1;
    if (node >= 0 && node < n_nodes) {
      const int x = node * ns + m % ns;
      c = a.stash ? kids_l[x] : kids[x];
    }
    c = (c >= 0 && c < visible) ? c : -1;
    const uint32_t bit = 1u << (c & 31);
    cand[n_fresh + m] = (c >= 0 && !(atomicOr(&seen[c >> 5], bit) & bit)) ? c : -1;
  }
  __syncthreads();
  const int k = min(a.K, a.cand_pow2);
  if (fresh_ahead) {
    score_keys<CT, SPAN>(qs, bcent, D, n_kids, [&](int m) { return cand[n_fresh + m]; }, keys + n_fresh);
  } else {
    score_keys<CT, SPAN>(qs, bcent, D, n_cand, [&](int j) { return cand[j]; }, keys);
  }
  for (int j = n_cand + tid; j < a.cand_pow2; j += LSA_BLOCK) keys[j] = 0;
  __syncthreads();
  block_topk_sorted(keys, a.cand_pow2, k, a.top_pow2, best, &sh.tks, &sh.st);
  for (int j = tid; j < a.K; j += LSA_BLOCK) {
    const int32_t b = j < k ? key_column(u_to_key(best[j])) : -1;
    sh.pick[j] = (b >= 0 && b < a.rows) ? b : -1;
  }
  __syncthreads();
  DECODE_MARK(4);
  publish_picks(a, sh, i, t, position, a.stash && ends ? ends_l : ends);
}

// The reader's work once it holds its unit's picks (sh.pick: a pick's bucket, or its first
// kept id for span tables; sh.start / sh.n: its first list slot and kept count; sh.filled):
// the unit's list of L = filled + tail slots is cut into tiles of `span` slots, and reader
// `role` takes a contiguous run of them (the first TT % NR readers one tile more), so only
// the last tile of a list is partial. The run is expanded into `ids` (and the list) in
// chunks of up to a.chunk tiles and read with the software-pipelined tile loop (its share
// of the list padding goes out first: it needs only the list's length, and stores issued
// before the gathers stay off the tail); then the reader publishes its split partial and
// arrives. The last reader of the unit combines the partials and leaves the unit's hand-off
// words zero for the next launch (`clear`: 1 the record copies, 2 the published keys).
// Tiles of an id chunk: a reader restarts its gather pipeline once a chunk, so the exchange
// and rank forms expand whole runs (B=32 x 32k flat 82.1 -> 81.0 us, B=32 x 131k tree
// 77.3 -> 76.5 with 32 against 8); the replicated form keeps 8 (its LDS holds the table).
constexpr int kChunkTiles = 32;
constexpr int kRepChunkTiles = 8;

// `map` turns a logical position into its cache row (a paged cache's slot table row of the
// unit's query row, loaded by the caller before its wait; the identity without one): the
// list and the gather hold mapped ids, while which ids are kept was decided on positions.
// A paged cache: reader `role` of the unit's NR readers touches its share of the 128-byte
// lines of the slot table row's entries [0, min(width, position + 1)) - one load a thread,
// at most LSA_BLOCK lines a reader - so the lines sit in the L2 of the XCD the unit runs on
// (every workgroup of a unit does) when the expansion maps its ids. Issued before the
// reader's wait; the caller consumes the value after it (keep_live), so nothing waits on it.
__device__ __forceinline__ int32_t touch_slot_lines(const SlotRow& map, int64_t position, int role, int NR) {
  if (map.row == nullptr) return 0;
  const int64_t lim = (int64_t)map.width < position + 1 ? (int64_t)map.width : position + 1;
  if (lim <= 0) return 0;
  const int64_t lines = (lim + 31) / 32;
  const int64_t per = (lines + NR - 1) / NR;
  const int64_t l = (int64_t)role * per + threadIdx.x;
  const int64_t e = l * 32 < lim ? l * 32 : lim - 1;  // in bounds whatever the lane
  const int32_t x = map.row[e];
  return threadIdx.x < per ? x : 0;
}

// Makes the compiler keep (and wait for) a value here without using it.
__device__ __forceinline__ void keep_live(int32_t x) { asm volatile("" ::"v"(x)); }

template <typename T, int D, int GQ>
__device__ __forceinline__ void read_parts(const DecodeArgs& a, RdLds<D, GQ>& sh, int32_t* ids, int64_t i, int role,
                                           const QueryRegs<T, D, GQ>& qr, int64_t position, int clear,
                                           const SlotRow map) {
  using S = ReadShape<T, D, GQ>;
  constexpr int VEC = S::VEC, LPT = S::LPT;
  constexpr int PSTRIDE = GQ * (D + 2);
  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1), w = tid / LSA_WAVE;
  const int K = a.K, span = a.span, words = 2 * K;
  const int64_t r = (uint32_t)i / (uint32_t)a.G;
  const int g = (int)((uint32_t)i % (uint32_t)a.G);
  const int64_t wstart = window_start_of(position, a.window);
  const int64_t n_win = position + 1 - wstart > 0 ? position + 1 - wstart : 0;
  const int64_t n_sink = a.sink < wstart ? a.sink : wstart;
  const int filled = sh.filled;
  const int length = filled + (int)(n_win + n_sink);
  const int TT = (length + span - 1) / span;  // tiles of the list
  const int NR = a.NR;
  const int q_t = TT / NR, rem = TT % NR;
  const int t_lo = role * q_t + (role < rem ? role : rem);
  const int t_hi = t_lo + q_t + (role < rem ? 1 : 0);
  const int lo = t_lo * span, hi = min(length, t_hi * span);
  const int n_part = TT < NR ? TT : NR;  // readers with a tile: roles [0, n_part)
  int32_t* lrow = a.lists + i * (int64_t)a.W;
  const int32_t* tab = a.members + (r * a.row_tables + g * a.group_tables) * (int64_t)a.rows * a.cap;
  const int lp = lane % LPT;
  const T* kb = (const T*)a.k + r * a.kv_sb + g * a.kv_sh + lp * VEC;
  const T* vb = (const T*)a.v + r * a.kv_sb + g * a.kv_sh + lp * VEC;
  // the last pick whose first slot is <= s (picks without slots share the next one's start)
  auto pick_of = [&](int s_) {
    int a_ = 0, b_ = K;
    while (b_ - a_ > 1) {
      const int m_ = (a_ + b_) >> 1;
      if (sh.start[m_] <= s_) a_ = m_; else b_ = m_;
    }
    return a_;
  };
  // the list's padding [length, W) is shared out over the unit's readers
  {
    const int per = (a.W - length + NR - 1) / NR;
    const int p0 = length + role * per;
    const int p1 = min(p0 + per, a.W);
    for (int k = p0 + tid; k < p1; k += LSA_BLOCK) lrow[k] = -1;
  }
  AttnState<T, D, GQ> st;
  st.clear();
  bool fresh = true;
  for (int c_lo = lo; c_lo < hi; c_lo += a.chunk * span) {
    const int c_hi = min(hi, c_lo + a.chunk * span);
    const int n = c_hi - c_lo;
    if (a.spans) {  // a pick's kept members are consecutive ids from the record's first one
      for (int k = tid; k < n; k += LSA_BLOCK) {
        const int s_ = c_lo + k;
        int32_t id;
        if (s_ < filled) {
          const int j = pick_of(s_);
          id = sh.pick[j] + (s_ - sh.start[j]);
        } else {
          id = tail_id(s_ - filled, wstart, n_win, n_sink);
        }
        id = map(id);
        ids[k] = id;
        lrow[s_] = id;
      }
    } else {
      for (int k = tid; k < n; k += LSA_BLOCK) {
        const int s_ = c_lo + k;
        if (s_ >= filled) {
          const int32_t id = map(tail_id(s_ - filled, wstart, n_win, n_sink));
          ids[k] = id;
          lrow[s_] = id;
        }
      }
      // the picks overlapping [c_lo, min(c_hi, filled)): ranks of each one's kept members in
      // table order, by a block ballot scan over its member row
      const uint64_t below = (1ull << lane) - 1ull;
      for (int s0 = c_lo; s0 < min(c_hi, filled);) {  // uniform over the block
        const int j = pick_of(s0);
        const int lo_rank = s0 - sh.start[j];
        const int nn = min(sh.start[j] + sh.n[j], c_hi) - s0;
        const int32_t* row = tab + (int64_t)sh.pick[j] * a.cap;
        for (int e0 = 0, run = 0; e0 < a.cap && run < lo_rank + nn; e0 += LSA_BLOCK) {
          const int e = e0 + tid;
          const int32_t id = row[e < a.cap ? e : 0];
          const bool keep = e < a.cap && id >= a.sink && (int64_t)id < wstart;
          const uint64_t m = __ballot(keep);
          if (lane == 0) sh.wcnt[w] = (int)__popcll(m);
          __syncthreads();
          int off = 0, tot = 0;
#pragma unroll
          for (int ww = 0; ww < LSA_WAVES; ++ww) {
            const int c = sh.wcnt[ww];
            off += ww < w ? c : 0;
            tot += c;
          }
          const int rank = run + off + (int)__popcll(m & below) - lo_rank;
          if (keep && rank >= 0 && rank < nn) {
            const int32_t m = map(id);
            ids[s0 - c_lo + rank] = m;
            lrow[s0 + rank] = m;
          }
          run += tot;
          __syncthreads();  // wcnt is rewritten by the next chunk of the row
        }
        s0 += nn;
      }
    }
    __syncthreads();
    DECODE_MARK(2);
    attend_tiles<T, D, GQ, true>(
        qr, kb, vb, a.kv_st, a.Tk, 0, n,
        [&](int jj) {
          const int32_t x = ids[jj < n ? jj : 0];
          return jj < n ? x : -1;
        },
        a.scale_log2, fresh, st);
    fresh = false;
    __syncthreads();  // ids are rewritten by the next chunk
    DECODE_MARK(3);
  }

  T* outp = (T*)a.out + (r * a.Hq + (int64_t)g * GQ) * D;
  float* parts = a.ws_part + i * (int64_t)a.NR * PSTRIDE;
  if (role < n_part) {
    finish_span<T, D, GQ>(sh.rd, st, n_part == 1, outp, n_part > 1 ? parts + (int64_t)role * PSTRIDE : nullptr, 0);
  }
  DECODE_MARK(4);
  if (!arrive_last(&a.rd_count[i], NR, &sh.rd.flag)) return;
  DECODE_MARK(5);
  if (n_part > 1) {
    combine_partials<T, D, GQ>(sh.rd, parts, n_part, outp, 0);
  } else if (n_part == 0) {  // nothing to read: zeros
    for (int k = tid; k < GQ * D; k += LSA_BLOCK) store_out<T>(outp + k, 0.0f);
  }
  if (clear == 1) {
    for (int x = tid; x < kRecordCopies * words; x += LSA_BLOCK) {
      const int c = x / words, k = x - c * words;
      coherent_store_i32(a.record + c * a.cstride + i * words + k, 0);
    }
  } else if (clear == 2) {
    uint64_t* mine = a.pub + i * (int64_t)a.rows;
    for (int x = tid; x < a.rows; x += LSA_BLOCK) coherent_store_u64(mine + x, 0);
  }
  DECODE_MARK(6);
}

// Wave 0 of a ranking reader: polls the unit's `rows` published keys (KPL a lane, all
// loads in flight each round) until every one is nonzero or the spin limit passes (*bad),
// then ranks them into rk->best (*fast, keys[] the candidate buffer): up to 32 picks by
// wave_topk_small (registers only, ~0.6 us faster at 512 keys), else, or when more than 64
// keys reach its bound, by wave_topk_sort; when a score is not finite the keys go to LDS
// for block_topk_sorted.
template <int KPL>
__device__ __forceinline__ void poll_and_rank(const DecodeArgs& a, const uint64_t* pub, int rows, uint64_t* keys,
                                              RankLds* rk, int* bad, int* fast) {
  const int lane = threadIdx.x & (LSA_WAVE - 1);
  uint64_t x[KPL];
  for (int it = 0;; ++it) {
    bool ok = true;
#pragma unroll
    for (int m = 0; m < KPL; ++m) {  // unconditional (clamped) loads: all in flight
      const int j = m * LSA_WAVE + lane;
      x[m] = coherent_load_u64(pub + (j < rows ? j : 0));
      ok &= j >= rows || x[m] != 0;
    }
    if (__all(ok)) break;
    if (it >= a.spin_limit) {
      *bad = 1;
      return;
    }
    __builtin_amdgcn_s_sleep(2);
  }
#pragma unroll
  for (int m = 0; m < KPL; ++m) x[m] = m * LSA_WAVE + lane < rows ? x[m] - 1 : 0;  // EMPTY past the table
  if ((a.K <= LSA_WAVE / 2 && wave_topk_small<KPL>(x, a.K, a.kp, rk->best, keys)) ||  // uniform
      wave_topk_sort<KPL>(x, a.K, a.kp, rk->best, keys, &rk->tks)) {
    *fast = 1;
    return;
  }
#pragma unroll
  for (int m = 0; m < KPL; ++m) {
    const int j = m * LSA_WAVE + lane;
    if (j < rows) keys[j] = x[m];
  }
}

// Reader of the rank form: no record. The unit's select splits publish their columns' keys
// (+ 1) and every reader ranks them itself: it loads its query rows (and a span table's
// ends), waits (bounded) until all `rows` published keys are nonzero, selects the K best
// (the last split's selection of the exchange form, on the same keys), counts each pick's
// kept members (span ends, or the member rows) and their list slots as publish_picks does,
// and reads its share. Role 0 writes the list length; the last reader clears the published
// keys.
template <typename T, int D, int GQ>
__device__ __forceinline__ void rank_reader(const DecodeArgs& a, char* smem, int64_t i, int role) {
  RdLds<D, GQ>& sh = *(RdLds<D, GQ>*)smem;
  RankLds& rk = *(RankLds*)(smem + rd_ids_offset<D, GQ>());
  int32_t* ends_l = (int32_t*)(smem + rank_ends_offset<D, GQ>());       // [rows]
  uint64_t* keys = (uint64_t*)(smem + rank_keys_offset<D, GQ>(a.rows));  // [rows]
  int32_t* ids = (int32_t*)(smem + rd_ids_offset<D, GQ>());              // after the selection
  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1), w = tid / LSA_WAVE;
  const int K = a.K, rows = a.rows;
  const int64_t r = (uint32_t)i / (uint32_t)a.G;
  const int g = (int)((uint32_t)i % (uint32_t)a.G);
  const int64_t position = a.positions[r];
  const int64_t wstart = window_start_of(position, a.window);
  const int64_t n_win = position + 1 - wstart > 0 ? position + 1 - wstart : 0;
  const int64_t n_sink = a.sink < wstart ? a.sink : wstart;
  const int64_t t = r * a.row_tables + g * a.group_tables;
  uint64_t* pub = a.pub + i * (int64_t)rows;
  DECODE_MARK(0);

  // the query rows, the slot table row and (span tables) the span ends go out before the wait
  const T* qrow = (const T*)a.q + (r * a.Hq + (int64_t)g * GQ) * D;
  QueryRegs<T, D, GQ> qr;
  qr.load(qrow, a.scale_log2);
  const SlotRow map = slot_row_of(a.slots, r);
  if (a.spans) {
    const int32_t* ends = a.ends + t * rows;
    for (int m = tid; m < rows; m += LSA_BLOCK) ends_l[m] = ends[m];
  }
  const int32_t touched = touch_slot_lines(map, position, role, a.NR);

  // wave 0 polls the published keys (every slot is nonzero once its split has written it)
  // and ranks them in its registers (wave_topk_hist); keys that defeat the histogram cut go
  // to LDS for the block's top-K
  if (w == 0) {
    int bad = 0, fast = 0;
    if (rows <= 8 * LSA_WAVE) poll_and_rank<8>(a, pub, rows, keys, &rk, &bad, &fast);
    else poll_and_rank<kRankKeysPerLane>(a, pub, rows, keys, &rk, &bad, &fast);
    if (lane == 0) {
      sh.bad = bad;
      rk.fast = fast;
      if (bad && a.status) __hip_atomic_store(a.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
  __syncthreads();
  DECODE_MARK(1);
  keep_live(touched);
  if (sh.bad) {  // no keys: this reader writes nothing but still arrives (see reader_role)
    if (arrive_last(&a.rd_count[i], a.NR, &sh.rd.flag)) {
      for (int x = tid; x < rows; x += LSA_BLOCK) coherent_store_u64(pub + x, 0);
    }
    return;
  }
  if (!rk.fast) block_topk_sorted(keys, rows, K, a.kp, rk.best, &rk.tks, &rk.st);
  // the picks (bucket rows, -1 = none); member tables count each pick's kept members from
  // its member row (count_members, the exchange form's count)
  const int32_t col = key_column(u_to_key(w == 0 && lane < K ? rk.best[lane] : 0));
  const int b = (w == 0 && lane < K && col >= 0 && col < rows) ? col : -1;
  if (!a.spans) {
    if (w == 0 && lane < K) sh.pick[lane] = b;
    __syncthreads();
    count_members(a, a.members + t * (int64_t)rows * a.cap, sh.pick, sh.n, wstart);
    __syncthreads();
  }
  // each pick's kept count (span tables: the range [max(begin, sink), min(end, window
  // start)) from the span ends) and its list slots
  if (w == 0) {
    int cnt = 0, first = b;
    if (a.spans) {
      const int64_t begin = b > 0 ? ends_l[b - 1] : 0, end_b = b >= 0 ? ends_l[b] : 0;
      const int64_t lo = begin > a.sink ? begin : a.sink, hi = end_b < wstart ? end_b : wstart;
      cnt = b >= 0 && hi > lo ? (int)(hi - lo) : 0;
      first = (int)lo;  // a pick's kept members are consecutive ids from here
    } else {
      cnt = lane < K ? sh.n[lane] : 0;
    }
    const int incl = wave_inclusive_sum(cnt);
    const int end = incl < a.top_k ? incl : a.top_k;
    int prev = dpp_or<kDppWaveShr1>(0, end);  // lane - 1's
    if (lane == 0) prev = 0;
    if (lane < K) {
      sh.pick[lane] = first;
      sh.start[lane] = prev;
      sh.n[lane] = end - prev;
    }
    const int filled = __builtin_amdgcn_readlane(end, K - 1);
    if (lane == 0) {
      sh.filled = filled;
      if (role == 0) a.lengths[i] = filled + (int)n_win + (int)n_sink;
    }
  }
  __syncthreads();
  DECODE_MARK(7);
  read_parts<T, D, GQ>(a, sh, ids, i, role, qr, position, 2, map);
}

template <typename T, int D, int GQ>
__device__ __forceinline__ void reader_role(const DecodeArgs& a, char* smem, int64_t i, int role) {
  using S = ReadShape<T, D, GQ>;
  constexpr int VEC = S::VEC, LPT = S::LPT;
  constexpr int PSTRIDE = GQ * (D + 2);
  RdLds<D, GQ>& sh = *(RdLds<D, GQ>*)smem;
  int32_t* ids = (int32_t*)(smem + rd_ids_offset<D, GQ>());  // [span]
  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1), w = tid / LSA_WAVE;
  const int K = a.K, span = a.span, words = 2 * K;
  const int64_t r = (uint32_t)i / (uint32_t)a.G;  // units < 2^31 (checked on the host): 32-bit division
  const int g = (int)((uint32_t)i % (uint32_t)a.G);
  const int64_t position = a.positions[r];
  const int64_t wstart = window_start_of(position, a.window);
  const int64_t n_win = position + 1 - wstart > 0 ? position + 1 - wstart : 0;
  const int64_t n_sink = a.sink < wstart ? a.sink : wstart;
  const int n_tail = (int)(n_win + n_sink);
  const int32_t* mine = a.record + (role % kRecordCopies) * a.cstride + i * words;
  DECODE_MARK(0);

  // the query rows and the slot table row go out before the wait
  const T* qrow = (const T*)a.q + (r * a.Hq + (int64_t)g * GQ) * D;
  QueryRegs<T, D, GQ> qr;
  qr.load(qrow, a.scale_log2);
  const SlotRow map = slot_row_of(a.slots, r);
  const int32_t touched = touch_slot_lines(map, position, role, a.NR);

  // wait for the unit's record; wave 0 polls its copy and decodes it
  if (w == 0) {
    int32_t wa = 1, wb = 1;
    int bad = 0;
    for (int it = 0;; ++it) {
      wa = lane < K ? coherent_load_i32(mine + lane) : 1;
      wb = lane < K ? coherent_load_i32(mine + K + lane) : 1;
      if (__all(wa != 0 && wb != 0)) break;
      if (it >= a.spin_limit) {
        bad = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    const int end = wb - 1;
    int prev = dpp_or<kDppWaveShr1>(0, end);  // lane - 1's
    if (lane == 0) prev = 0;
    const int n = lane < K ? end - prev : 0;
    if (lane < K) {
      sh.pick[lane] = wa - 2;
      sh.start[lane] = prev;
      sh.n[lane] = n;
    }
    const int filled = __builtin_amdgcn_readlane(end, K - 1);
    if (lane == 0) {
      sh.filled = filled;
      sh.bad = bad;
      if (bad && a.status) __hip_atomic_store(a.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
  __syncthreads();
  DECODE_MARK(1);
  keep_live(touched);
  if (sh.bad) {
    // no record: this reader writes nothing but still arrives, so the unit's counter
    // resets; *status tells the caller the unit's outputs are invalid
    if (arrive_last(&a.rd_count[i], a.NR, &sh.rd.flag)) {
      for (int x = tid; x < kRecordCopies * words; x += LSA_BLOCK) {
        const int c = x / words, k = x - c * words;
        coherent_store_i32(a.record + c * a.cstride + i * words + k, 0);
      }
    }
    return;
  }

  read_parts<T, D, GQ>(a, sh, ids, i, role, qr, position, 1, map);
}

// ------------------------------------------------------------------ replicated select

// Every reader workgroup selects for itself (no select workgroups, no cross-workgroup wait
// before the gather): it screens its unit's whole table on the matrix cores and re-scores
// the rows near the cut exactly (screen_topk: the canonical top-K, ties to the lower
// bucket). Every reader of a unit computes the same picks (identical inputs and
// instruction sequence). Span tables, bf16 scoring, head dim 32/64/128, at most
// kScreenMaxRows buckets and 64 picks.
constexpr int kRepMaxRows = kScreenMaxRows;

struct RepLds {
  ScreenLds scr;
  int32_t ends[kRepMaxRows];  // the table's span ends
  uint64_t best[kMaxPicks];
};

template <int D, int GQ>
constexpr size_t rep_extra_offset() {
  return (sizeof(RdLds<D, GQ>) + 15) & ~(size_t)15;
}
template <int D, int GQ>
constexpr size_t rep_ids_offset() {
  return (rep_extra_offset<D, GQ>() + sizeof(RepLds) + 15) & ~(size_t)15;
}

template <typename T, int D, int GQ>
__device__ __forceinline__ void rep_role(const DecodeArgs& a, char* smem, int64_t i, int role) {
  constexpr int SPAN = D / 16;
  RdLds<D, GQ>& sh = *(RdLds<D, GQ>*)smem;
  RepLds& ex = *(RepLds*)(smem + rep_extra_offset<D, GQ>());
  int32_t* ids = (int32_t*)(smem + rep_ids_offset<D, GQ>());
  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1), w = tid / LSA_WAVE;
  const int K = a.K, rows = a.rows;
  const int64_t r = (uint32_t)i / (uint32_t)a.G;
  const int g = (int)((uint32_t)i % (uint32_t)a.G);
  const int64_t position = a.positions[r];
  const int64_t t = r * a.row_tables + g * a.group_tables;
  const bf16_t* cent = (const bf16_t*)a.centroids + t * (int64_t)rows * D;
  const int32_t* ends = a.ends + t * rows;
  const int64_t lim = position + 1;
  const int64_t wstart = window_start_of(position, a.window);
  const T* qrow = (const T*)a.q + (r * a.Hq + (int64_t)g * GQ) * D;
  DECODE_MARK(8);

  // the span ends into LDS, the query rows for the read, the index query (the group mean,
  // bf16-rounded, in the 16-lane layout)
  for (int m = tid; m < rows; m += LSA_BLOCK) ex.ends[m] = ends[m];
  QueryRegs<T, D, GQ> qr;
  qr.load(qrow, a.scale_log2);
  const SlotRow map = slot_row_of(a.slots, r);
  float qs[SPAN];
  group_mean_slice<T, SPAN, GQ>(qrow, tid & 15, true, qs);
  __syncthreads();  // the span ends in LDS
  screen_topk<D, 2>(
      qs, cent, rows, [](int j) { return j; }, [&](int j) { return (int64_t)ex.ends[j] <= lim; }, K, a.kp, ex.best,
      ex.scr);
  DECODE_MARK(11);
  if (w == 0) {
    const uint64_t v = lane < a.kp ? ex.best[lane] : 0;
    const int32_t b = key_column(u_to_key(v));
    sh.pick[lane] = (lane < K && b >= 0 && b < rows) ? b : -1;
  }
  __syncthreads();

  // each pick's kept range [max(begin, sink), min(end, window start)) and its list slots
  // (as the record of the exchange form gives them)
  if (w == 0) {
    const int b = lane < K ? sh.pick[lane] : -1;
    int cntk = 0, first = 0;
    if (b >= 0) {
      const int64_t begin = b > 0 ? ex.ends[b - 1] : 0, end = ex.ends[b];
      const int64_t lo = begin > a.sink ? begin : a.sink, hi = end < wstart ? end : wstart;
      cntk = hi > lo ? (int)(hi - lo) : 0;
      first = (int)lo;
    }
    const int incl = wave_inclusive_sum(cntk);
    const int end = incl < a.top_k ? incl : a.top_k;
    int prev = dpp_or<kDppWaveShr1>(0, end);  // lane - 1's
    if (lane == 0) prev = 0;
    const int n = lane < K ? end - prev : 0;
    if (lane < K) {
      sh.pick[lane] = first;
      sh.start[lane] = prev;
      sh.n[lane] = n;
    }
    const int filled = __builtin_amdgcn_readlane(end, K - 1);
    if (lane == 0) {
      sh.filled = filled;
      if (role == 0) {
        const int64_t n_win = position + 1 - wstart > 0 ? position + 1 - wstart : 0;
        const int64_t n_sink = a.sink < wstart ? a.sink : wstart;
        a.lengths[i] = filled + (int)n_win + (int)n_sink;
      }
    }
  }
  __syncthreads();
  read_parts<T, D, GQ>(a, sh, ids, i, role, qr, position, 0, map);
}

// One workgroup per (unit, reader), unit fastest: every workgroup is a reader that
// selects for itself (rep_role).
template <typename T, int D, int GQ>
__global__ __launch_bounds__(LSA_BLOCK) void decode_rep_kernel(DecodeArgs a) {
  extern __shared__ __align__(16) char smem[];
  const uint32_t units = (uint32_t)(a.R * a.G);  // the grid is < 2^31 workgroups (checked on the host)
  const uint32_t id = blockIdx.x;
  DECODE_TRACE_BEGIN();
  rep_role<T, D, GQ>(a, smem, id % units, (int)(id / units));
  DECODE_TRACE_END();
}

template <typename T, typename CT, int D, int GQ>
__global__ __launch_bounds__(LSA_BLOCK) void decode_flat_kernel(DecodeArgs a) {
  extern __shared__ __align__(16) char smem[];
  const uint32_t units = (uint32_t)(a.R * a.G);  // the grid is < 2^31 workgroups (checked on the host)
  const uint32_t id = blockIdx.x;
  const uint32_t nsel = units * (uint32_t)a.S;
  DECODE_TRACE_BEGIN();
  if (id < nsel) {
    if (a.tree) tree_role<T, CT, D, GQ>(a, smem, id);  // one select workgroup a unit
    else select_role<T, CT, D, GQ>(a, smem, id % units, (int)(id / units));
  } else {
    const uint32_t rid = id - nsel;  // readers: unit fastest, then role (low roles have work)
    if (a.rank) rank_reader<T, D, GQ>(a, smem, rid % units, (int)(rid / units));
    else reader_role<T, D, GQ>(a, smem, rid % units, (int)(rid / units));
  }
  DECODE_TRACE_END();
}

// ------------------------------------------------------------------ launch

template <typename T, typename CT, int D, int GQ>
void launch_one(const DecodeArgs& a, bool rep, dim3 grid, size_t shmem, hipStream_t s) {
  if constexpr (D <= 128 && __is_same(CT, bf16_t)) {
    if (rep) {
      decode_rep_kernel<T, D, GQ><<<grid, LSA_BLOCK, shmem, s>>>(a);
      return;
    }
  }
  decode_flat_kernel<T, CT, D, GQ><<<grid, LSA_BLOCK, shmem, s>>>(a);
}

template <typename T, typename CT, int D>
void launch_gq(const DecodeArgs& a, bool rep, int gq, dim3 grid, size_t shmem, hipStream_t s) {
  switch (gq) {
    case 1: launch_one<T, CT, D, 1>(a, rep, grid, shmem, s); break;
    case 2: launch_one<T, CT, D, 2>(a, rep, grid, shmem, s); break;
    case 4: launch_one<T, CT, D, 4>(a, rep, grid, shmem, s); break;
    default: launch_one<T, CT, D, 8>(a, rep, grid, shmem, s); break;
  }
}

template <typename T, typename CT>
void launch_d(const DecodeArgs& a, bool rep, int D, int gq, dim3 grid, size_t shmem, hipStream_t s) {
  switch (D) {
    case 32: launch_gq<T, CT, 32>(a, rep, gq, grid, shmem, s); break;
    case 64: launch_gq<T, CT, 64>(a, rep, gq, grid, shmem, s); break;
    case 128: launch_gq<T, CT, 128>(a, rep, gq, grid, shmem, s); break;
    default: launch_gq<T, CT, 256>(a, rep, gq, grid, shmem, s); break;
  }
}

// rep: the replicated-select kernel (bf16 tables, D <= 128); else the exchange kernel.
template <typename T>
void launch_type(const DecodeArgs& a, bool rep, bool bf16_table, int D, int gq, dim3 grid, size_t shmem,
                 hipStream_t s) {
  if (bf16_table) launch_d<T, bf16_t>(a, rep, D, gq, grid, shmem, s);
  else launch_d<T, float>(a, false, D, gq, grid, shmem, s);
}

// Defined by decode_bf16.hip, decode_f16.hip and decode_f32.hip.
void launch_bf16(const DecodeArgs& a, bool rep, bool bf16_table, int D, int gq, dim3 grid, size_t shmem,
                 hipStream_t s);
void launch_f16(const DecodeArgs& a, bool rep, bool bf16_table, int D, int gq, dim3 grid, size_t shmem,
                hipStream_t s);
void launch_f32(const DecodeArgs& a, bool rep, bool bf16_table, int D, int gq, dim3 grid, size_t shmem,
                hipStream_t s);

}  // namespace decode
}  // namespace lsa
