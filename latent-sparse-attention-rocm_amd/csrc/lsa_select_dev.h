// Selection device code: canonical scoring, visibility, top-k and the rank-order
// expansion walk, shared by the standalone and the fused select kernels.
#pragma once

#include "lsa_device.h"

namespace lsa {

// A contiguous stack of bucket tables; table t = r * row_tables + g * group_tables.
struct Tables {
  const void* centroids;   // [tables, rows, dim] bf16 (bf16 scoring) or fp32 (fp32 scoring)
  const int32_t* members;  // [tables, rows, cap], -1 padded
  const int32_t* ends;     // [tables, rows] exclusive span ends (nondecreasing) or nullptr
  int64_t row_tables;      // tables between query rows (0: every row shares)
  int64_t group_tables;    // tables between groups (0: every group shares)
  int32_t rows;            // buckets per table
  int32_t cap;             // member slots per bucket
  int32_t dim;             // index dim
};

__device__ __forceinline__ int64_t table_of(const Tables& t, int64_t r, int64_t g) {
  return r * t.row_tables + g * t.group_tables;
}

// Buckets a query at `position` scores (reference pipeline.py:184-186): the closed
// cluster blocks before it, or with span ends the buckets ending at or before pos+1.
__device__ __forceinline__ int visible_count(int64_t position, int rows, int cluster_block, int block_buckets,
                                             const int32_t* ends) {
  if (ends == nullptr) {
    int64_t blocks = position >= 0 ? position / cluster_block : -((-position + cluster_block - 1) / cluster_block);
    int64_t v = blocks * block_buckets;
    if (v > rows) v = rows;
    return (int)v;  // may be negative: nothing visible
  }
  // upper bound: first index with ends[i] > position + 1
  int lo = 0, hi = rows;
  const int64_t lim = position + 1;
  while (lo < hi) {
    int mid = (lo + hi) >> 1;
    if ((int64_t)ends[mid] <= lim) lo = mid + 1; else hi = mid;
  }
  return lo;
}

// Loads one lane's slice of a query row, rounded to the scoring type.
template <typename QT, int SPAN>
__device__ __forceinline__ void load_query_slice(const QT* q, int p, bool bf16_mode, float* out) {
#pragma unroll
  for (int j = 0; j < SPAN; ++j) {
    float x = elem<QT>::load(q, (int64_t)p * SPAN + j);
    out[j] = bf16_mode ? bf16_round(x) : x;
  }
}

// fp64 partial over the lane's slice, then the 16-lane tree: the canonical score.
template <typename CT, int SPAN>
__device__ __forceinline__ float canonical_score(const float* qs, const CT* row, int p) {
  double acc = 0.0;
  const CT* base = row + (int64_t)p * SPAN;
#pragma unroll
  for (int j = 0; j < SPAN; ++j) acc = fma((double)qs[j], (double)elem<CT>::load(base, j), acc);
  return score_tree16(acc);
}

// Scores columns [c0, c1) of one table into u-ordered keys out[c - c0]; columns at or
// past `visible` become EMPTY (u == 0). Every thread of the block calls it.
template <typename CT, int SPAN>
__device__ void score_slice_keys(const float* qs, const CT* cent, int dim, int c0, int c1, int visible,
                                 uint64_t* out) {
  const int grp = threadIdx.x >> 4, p = threadIdx.x & 15;
  for (int c = c0 + grp; c < c1; c += LSA_BLOCK / 16) {
    uint64_t u = 0;
    if (c < visible) {  // uniform over the 16-lane group
      float s = canonical_score<CT, SPAN>(qs, cent + (int64_t)c * dim, p);
      u = key_to_u(pack_key(s, c));
    }
    if (p == 0) out[c - c0] = u;
  }
}

// Rank-order expansion of one row (reference select_fused.py:172-214): picks in rank
// order, member slots in table order, keep ids with sink <= id < window_start until
// top_k are stored; then the window [window_start, position] and the sinks
// [0, min(sink, window_start)). Slots past the length are -1. Returns the length.
// picks lives in LDS (bucket ids, -1 = none). Every thread of the block calls it.
__device__ int expand_walk(const int32_t* picks, int n_picks, const int32_t* members, int rows, int cap,
                           int64_t position, int window, int sink, int top_k, int32_t* out, int width,
                           int* scan) {
  constexpr int E = 8;  // consecutive slots per thread per tile
  const int tid = threadIdx.x;
  int64_t ws = position + 1 - window;
  const int64_t window_start = ws > 0 ? ws : 0;
  const int64_t total_slots = (int64_t)n_picks * cap;
  int filled = 0;
  for (int64_t base = 0; base < total_slots && filled < top_k; base += (int64_t)LSA_BLOCK * E) {
    int32_t ids[E];
    int count = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int64_t s = base + (int64_t)tid * E + e;
      int32_t id = -1;
      if (s < total_slots) {
        const int32_t b = picks[s / cap];
        if (b >= 0 && b < rows) id = members[(int64_t)b * cap + (s % cap)];
      }
      const bool ok = (id >= sink) && ((int64_t)id < window_start);
      ids[e] = ok ? id : -1;
      count += ok ? 1 : 0;
    }
    int total;
    int at = filled + block_exclusive_sum(count, scan, &total);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if (ids[e] >= 0) {
        if (at < top_k) out[at] = ids[e];
        ++at;
      }
    }
    filled += total;
  }
  if (filled > top_k) filled = top_k;
  const int64_t n_win = position + 1 - window_start > 0 ? position + 1 - window_start : 0;
  const int64_t n_sink = sink < window_start ? sink : window_start;
  const int length = filled + (int)n_win + (int)n_sink;
  for (int i = tid; i < width - filled; i += LSA_BLOCK) {
    const int at = filled + i;
    int32_t v = -1;
    if (i < n_win) v = (int32_t)(window_start + i);
    else if (i < n_win + n_sink) v = (int32_t)(i - n_win);
    out[at] = v;
  }
  return length;
}

// Merges S descending lists (each K long, u-ordered, u == 0 padding) into the best K,
// descending, by rank: an element's rank is its index plus, for every other list, the
// number of its elements that beat it (ties to the lower list). Every thread calls it.
__device__ void merge_sorted_lists(const uint64_t* lists, int S, int K, uint64_t* out) {
  const int total = S * K;
  for (int e = threadIdx.x; e < total; e += LSA_BLOCK) {
    const int s = e / K, j = e % K;
    const uint64_t x = lists[e];
    int rank = j;
    for (int o = 0; o < S; ++o) {
      if (o == s) continue;
      const uint64_t* l = lists + (int64_t)o * K;
      // count of elements in l that beat x: > x, or >= x when o < s
      int lo = 0, hi = K;
      while (lo < hi) {
        int mid = (lo + hi) >> 1;
        bool beats = (o < s) ? (l[mid] >= x) : (l[mid] > x);
        if (beats) lo = mid + 1; else hi = mid;
      }
      rank += lo;
    }
    if (rank < K) out[rank] = x;
  }
  __syncthreads();
}

}  // namespace lsa
