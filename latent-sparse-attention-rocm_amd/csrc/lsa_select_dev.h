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


// visible_count for span ends, by the whole block in two rounds of parallel loads instead
// of a serial binary search (one dependent round trip per halving): thread t samples the
// end of stride-sized run t, the count of samples <= position + 1 names the run holding
// the boundary, and that run's ends are loaded and counted. `lds` holds 2 * LSA_WAVES
// ints. Every thread calls it; every thread gets the count.
__device__ __forceinline__ int visible_count_block(int64_t position, int rows, const int32_t* ends, int* lds) {
  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1), w = tid / LSA_WAVE;
  const int64_t lim = position + 1;
  const int step = (rows + LSA_BLOCK - 1) / LSA_BLOCK;  // ends per run (rows <= 256 * step)
  const int runs = (rows + step - 1) / step;
  const int s = min(rows - 1, (tid + 1) * step - 1);
  const bool le = tid < runs && (int64_t)ends[s] <= lim;  // run tid lies wholly at or below lim
  const int c1 = (int)__popcll(__ballot(le));  // every lane votes
  if (lane == 0) lds[w] = c1;
  __syncthreads();
  const int full = lds[0] + lds[1] + lds[2] + lds[3];  // runs wholly visible (ends are nondecreasing)
  const int base = min(full * step, rows);  // the last run may be short
  const int j = base + tid;
  const bool v2 = tid < step && j < rows && (int64_t)ends[j < rows ? j : rows - 1] <= lim;
  const int c2 = (int)__popcll(__ballot(v2));
  if (lane == 0) lds[LSA_WAVES + w] = c2;
  __syncthreads();
  return base + lds[LSA_WAVES] + lds[LSA_WAVES + 1] + lds[LSA_WAVES + 2] + lds[LSA_WAVES + 3];
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

// SPAN consecutive elements of a centroid row, loaded raw with the widest aligned vector
// loads (a lane's slice starts at a multiple of SPAN elements of a row whose length is
// 16 * SPAN elements, so SPAN * sizeof(CT) bytes of alignment hold for an aligned table).
template <typename CT, int SPAN>
struct SpanRaw {
  static constexpr int BYTES = SPAN * (int)sizeof(CT);
  static constexpr int WORDS = BYTES >= 4 ? BYTES / 4 : 1;
  uint32_t w[WORDS];
  __device__ __forceinline__ void load(const CT* p) {
    if constexpr (BYTES >= 16) {
#pragma unroll
      for (int i = 0; i < BYTES / 16; ++i) {
        const uint4 v = ((const uint4*)p)[i];
        w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
      }
    } else if constexpr (BYTES == 8) {
      const uint2 v = *(const uint2*)p;
      w[0] = v.x; w[1] = v.y;
    } else if constexpr (BYTES == 4) {
      w[0] = *(const uint32_t*)p;
    } else {
      w[0] = *(const uint16_t*)p;
    }
  }
  __device__ __forceinline__ float at(int j) const {
    if constexpr (sizeof(CT) == 4) {
      return __uint_as_float(w[j]);
    } else if constexpr (__is_same(CT, _Float16)) {
      const uint16_t h = (uint16_t)((j & 1) ? (w[j >> 1] >> 16) : (w[j >> 1] & 0xFFFFu));
      _Float16 f;
      __builtin_memcpy(&f, &h, 2);
      return (float)f;
    } else {  // bf16
      const uint32_t x = w[j >> 1];
      return __uint_as_float((j & 1) ? (x & 0xFFFF0000u) : (x << 16));
    }
  }
};

// Loads one lane's slice of a query row (all loads first), rounded to the scoring type.
template <typename QT, int SPAN>
__device__ __forceinline__ void load_query_slice(const QT* q, int p, bool bf16_mode, float* out) {
  SpanRaw<QT, SPAN> raw;
  raw.load(q + (int64_t)p * SPAN);
#pragma unroll
  for (int j = 0; j < SPAN; ++j) {
    const float x = raw.at(j);
    out[j] = bf16_mode ? bf16_round(x) : x;
  }
}

// One batch size of score_keys: each 16-lane group scores CB columns per round trip.
template <typename CT, int SPAN, int CB, typename ColOf, typename KeepOf>
__device__ __forceinline__ void score_keys_cb(const float* qs, const CT* cent, int dim, int n, ColOf col_of,
                                              KeepOf keep_of, uint64_t* out) {
  constexpr int GROUPS = LSA_BLOCK / 16;
  const int grp = threadIdx.x >> 4, p = threadIdx.x & 15;
  for (int jb = 0; jb < n; jb += GROUPS * CB) {
    SpanRaw<CT, SPAN> raw[CB];
    int col[CB];
    bool keep[CB];
#pragma unroll
    for (int k = 0; k < CB; ++k) {
      const int j = jb + k * GROUPS + grp;
      col[k] = j < n ? col_of(j) : -1;
      raw[k].load(cent + (int64_t)(col[k] >= 0 ? col[k] : 0) * dim + p * SPAN);
      keep[k] = keep_of(j < n ? j : n - 1) && j < n;
    }
#pragma unroll
    for (int k = 0; k < CB; ++k) {
      const int j = jb + k * GROUPS + grp;
      double acc = 0.0;
#pragma unroll
      for (int e = 0; e < SPAN; ++e) acc = fma((double)qs[e], (double)raw[k].at(e), acc);
      const float s = score_tree16(acc);
      if (p == 0 && j < n) out[j] = (col[k] >= 0 && keep[k]) ? key_to_u(pack_key(s, col[k])) : 0;
    }
  }
}

// Scores entries j < n of a column list into u-ordered keys out[j]: col_of(j) is a
// column of `cent` or -1 (EMPTY key, u == 0), keep_of(j) masks a scored column to EMPTY
// (its load is issued with the centroid rows, so it costs no extra round trip). Each
// 16-lane group scores one column per step; a batch of columns (sized to n, at most 256
// bytes of rows per lane) is loaded unconditionally (invalid ones read row 0) before any
// arithmetic, so a batch costs one memory round trip. Every thread calls it.
template <typename CT, int SPAN, typename ColOf, typename KeepOf>
__device__ __forceinline__ void score_keys(const float* qs, const CT* cent, int dim, int n, ColOf col_of,
                                           KeepOf keep_of, uint64_t* out) {
  constexpr int GROUPS = LSA_BLOCK / 16;
  constexpr int BYTES = SPAN * (int)sizeof(CT);
  constexpr int CBMAX = BYTES >= 256 ? 1 : (256 / BYTES > 16 ? 16 : 256 / BYTES);
  if (n <= GROUPS) score_keys_cb<CT, SPAN, 1>(qs, cent, dim, n, col_of, keep_of, out);
  else if (n <= 2 * GROUPS || CBMAX < 4) score_keys_cb<CT, SPAN, (CBMAX < 2 ? CBMAX : 2)>(qs, cent, dim, n, col_of, keep_of, out);
  else if (n <= 4 * GROUPS || CBMAX < 8) score_keys_cb<CT, SPAN, (CBMAX < 4 ? CBMAX : 4)>(qs, cent, dim, n, col_of, keep_of, out);
  else if (n <= 8 * GROUPS || CBMAX < 16) score_keys_cb<CT, SPAN, (CBMAX < 8 ? CBMAX : 8)>(qs, cent, dim, n, col_of, keep_of, out);
  else score_keys_cb<CT, SPAN, CBMAX>(qs, cent, dim, n, col_of, keep_of, out);
}

template <typename CT, int SPAN, typename ColOf>
__device__ __forceinline__ void score_keys(const float* qs, const CT* cent, int dim, int n, ColOf col_of,
                                           uint64_t* out) {
  score_keys<CT, SPAN>(qs, cent, dim, n, col_of, [](int) { return true; }, out);
}

// Scores columns [c0, c1) of one table into u-ordered keys out[c - c0]; columns at or
// past `visible` become EMPTY (u == 0). Every thread of the block calls it.
template <typename CT, int SPAN>
__device__ __forceinline__ void score_slice_keys(const float* qs, const CT* cent, int dim, int c0, int c1,
                                                 int visible, uint64_t* out) {
  const int n = c1 > c0 ? c1 - c0 : 0;
  score_keys<CT, SPAN>(qs, cent, dim, n, [&](int j) { return c0 + j < visible ? c0 + j : -1; }, out);
}

// Shared state of the histogram top-k (one per workgroup, in LDS).
constexpr int kTopBins = 512;       // bins of the binned top-K (large K)
constexpr int kTopBinsWide = 2048;  // the same for tables of thousands of keys (smaller bins to rank)

struct TopkScratch {
  int hist[256];
  int off[256];   // first candidate slot of each bin (bins from the top down)
  int fill[256];  // candidates placed so far per bin
  uint64_t cand[LSA_WAVE];
  float wmin[LSA_WAVES], wmax[LSA_WAVES];
  int wcnt[LSA_WAVES], wbad[LSA_WAVES];
  int cut, ok;
};

// State of block_topk_bins (large K), in LDS: keys a bin holds (counted down again as the
// candidates are placed) and the keys in the bins above it (bins in descending order).
template <int NB>
struct BinScratchN {
  int bcnt[NB], boff[NB];
  int wsum[LSA_WAVES], wocc[LSA_WAVES];
  int bcut, bnc, btot;
};
using BinScratch = BinScratchN<kTopBins>;
using BinScratchWide = BinScratchN<kTopBinsWide>;

// The score a u-ordered key was packed from (inverse of ordered_bits).
__device__ __forceinline__ float key_score(uint64_t u) {
  const int32_t ob = (int32_t)((uint32_t)(u >> 32) ^ 0x80000000u);
  return __int_as_float(ob ^ ((ob >> 31) & 0x7FFFFFFF));
}

// Histogram cut for a small K (<= 64). The nonempty keys are binned linearly by score over
// [min, max] into 256 bins (a monotone map: a higher bin never holds a lower key). The bins
// from the top down to the one holding the min(K, nonempty)-th key are the candidates;
// each is placed at its bin's offset (bins in descending order), so its rank is that
// offset plus the larger keys of its own bin - usually none. Returns false (every thread)
// when a score is not finite or more than 64 keys survive the cut (ties, a degenerate
// spread); the caller then uses the radix select. Every thread calls it. Designed for
// latency: five barriers and no loop longer than a bin's occupancy.
__device__ __forceinline__ bool block_topk_hist(const uint64_t* keys, int n, int K, int kp, uint64_t* out,
                                                TopkScratch* sc) {
  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1), w = tid / LSA_WAVE;
  float mn = INFINITY, mx = -INFINITY;
  int cnt = 0, bad = 0;
  for (int j = tid; j < n; j += LSA_BLOCK) {
    const uint64_t k = keys[j];
    const float x = key_score(k);
    const bool live = k != 0;
    bad |= (live && x - x != 0.0f) ? 1 : 0;  // NaN or infinite
    mn = live ? fminf(mn, x) : mn;
    mx = live ? fmaxf(mx, x) : mx;
    cnt += live ? 1 : 0;
  }
  sc->hist[tid] = 0;  // LSA_BLOCK == 256 bins
  sc->fill[tid] = 0;
  mn = wave_min(mn);
  mx = wave_max(mx);
  cnt = wave_sum(cnt);
  bad = wave_or(bad);
  if (lane == 0) { sc->wmin[w] = mn; sc->wmax[w] = mx; sc->wcnt[w] = cnt; sc->wbad[w] = bad; }
  __syncthreads();
  mn = fminf(fminf(sc->wmin[0], sc->wmin[1]), fminf(sc->wmin[2], sc->wmin[3]));
  mx = fmaxf(fmaxf(sc->wmax[0], sc->wmax[1]), fmaxf(sc->wmax[2], sc->wmax[3]));
  cnt = sc->wcnt[0] + sc->wcnt[1] + sc->wcnt[2] + sc->wcnt[3];
  bad = sc->wbad[0] | sc->wbad[1] | sc->wbad[2] | sc->wbad[3];
  if (bad) return false;  // uniform: every thread sees the same totals
  const int kc = cnt < K ? cnt : K;
  const float scale = mx > mn ? 256.0f / (mx - mn) : 0.0f;
  auto bin_of = [&](uint64_t k) {
    const int b = (int)((key_score(k) - mn) * scale);
    return b < 0 ? 0 : (b > 255 ? 255 : b);
  };
  for (int j = tid; j < n; j += LSA_BLOCK) {
    const uint64_t k = keys[j];
    if (k != 0) atomicAdd(&sc->hist[bin_of(k)], 1);
  }
  __syncthreads();
  if (w == 0) {
    // lane l owns bins 255-4l .. 252-4l; exclusive suffix offsets from the top bin
    const int c0 = sc->hist[255 - 4 * lane], c1 = sc->hist[254 - 4 * lane];
    const int c2 = sc->hist[253 - 4 * lane], c3 = sc->hist[252 - 4 * lane];
    const int mine = c0 + c1 + c2 + c3;
    const int inc = wave_inclusive_sum(mine);
    const int o0 = inc - mine, o1 = o0 + c0, o2 = o1 + c1, o3 = o2 + c2;
    sc->off[255 - 4 * lane] = o0;
    sc->off[254 - 4 * lane] = o1;
    sc->off[253 - 4 * lane] = o2;
    sc->off[252 - 4 * lane] = o3;
    // the bin holding the kc-th key, and the keys in it and above
    const bool here = kc > 0 && o0 < kc && kc <= inc;
    const int d = o1 >= kc ? 255 - 4 * lane : (o2 >= kc ? 254 - 4 * lane : (o3 >= kc ? 253 - 4 * lane : 252 - 4 * lane));
    const int total = o1 >= kc ? o1 : (o2 >= kc ? o2 : (o3 >= kc ? o3 : inc));
    const uint64_t m = __ballot(here);
    const int src = m ? __ffsll((long long)m) - 1 : 0;
    const int cut = __builtin_amdgcn_readlane(d, src);  // src is the same in every lane
    const int tot = __builtin_amdgcn_readlane(total, src);
    if (lane == 0) { sc->cut = m ? cut : 256; sc->ok = (m == 0 || tot <= LSA_WAVE) ? 1 : 0; }
  }
  __syncthreads();
  if (!sc->ok) return false;
  const int cut = sc->cut;
  for (int j = tid; j < n; j += LSA_BLOCK) {
    const uint64_t k = keys[j];
    const int b = bin_of(k);
    if (k != 0 && b >= cut) sc->cand[sc->off[b] + atomicAdd(&sc->fill[b], 1)] = k;
  }
  __syncthreads();
  if (w == 0) {
    const int nc = cut < 256 ? sc->off[cut] + sc->hist[cut] : 0;
    if (lane < nc) {
      const uint64_t x = sc->cand[lane];
      const int b = bin_of(x);
      const int lo = sc->off[b], hi = lo + sc->hist[b];
      int rank = lo;
      for (int m = lo; m < hi; ++m) rank += sc->cand[m] > x ? 1 : 0;  // nonempty keys are distinct
      if (rank < K) out[rank] = x;
    }
    for (int m = kc + lane; m < kp; m += LSA_WAVE) out[m] = 0;  // EMPTY past the nonempty keys
  }
  __syncthreads();
  return true;
}

// The histogram cut of block_topk_hist run by one wave on keys held in its registers, with
// no block barrier: x[m] is key m * LSA_WAVE + lane (u-ordered, 0 = EMPTY). The same bins,
// cut and ranking, so the same out[0..kp) (the K best sorted descending, EMPTY past them).
// sc->hist and sc->fill must be zero on entry (the wave clears them ahead of time). Returns
// false (in every lane) when a score is not finite or more than 64 keys survive the cut;
// the caller then takes block_topk_sorted. The wave's LDS accesses run in program order,
// and wave_barrier keeps the compiler from moving them across the phases.
template <int KPL>
__device__ __forceinline__ bool wave_topk_hist(const uint64_t* x, int K, int kp, uint64_t* out, TopkScratch* sc) {
  const int lane = threadIdx.x & (LSA_WAVE - 1);
  float mn = INFINITY, mx = -INFINITY;
  int cnt = 0, bad = 0;
#pragma unroll
  for (int m = 0; m < KPL; ++m) {
    const float s = key_score(x[m]);
    const bool live = x[m] != 0;
    bad |= (live && s - s != 0.0f) ? 1 : 0;  // NaN or infinite
    mn = live ? fminf(mn, s) : mn;
    mx = live ? fmaxf(mx, s) : mx;
    cnt += live ? 1 : 0;
  }
  mn = wave_min(mn);
  mx = wave_max(mx);
  cnt = wave_sum(cnt);
  if (wave_or(bad)) return false;
  const int kc = cnt < K ? cnt : K;
  const float scale = mx > mn ? 256.0f / (mx - mn) : 0.0f;
  auto bin_of = [&](uint64_t k) {
    const int b = (int)((key_score(k) - mn) * scale);
    return b < 0 ? 0 : (b > 255 ? 255 : b);
  };
  int bin[KPL];
#pragma unroll
  for (int m = 0; m < KPL; ++m) {
    bin[m] = bin_of(x[m]);
    if (x[m] != 0) atomicAdd(&sc->hist[bin[m]], 1);
  }
  __builtin_amdgcn_wave_barrier();
  // lane l owns bins 255-4l .. 252-4l; exclusive suffix offsets from the top bin
  const int c0 = sc->hist[255 - 4 * lane], c1 = sc->hist[254 - 4 * lane];
  const int c2 = sc->hist[253 - 4 * lane], c3 = sc->hist[252 - 4 * lane];
  const int mine = c0 + c1 + c2 + c3;
  const int inc = wave_inclusive_sum(mine);
  const int o0 = inc - mine, o1 = o0 + c0, o2 = o1 + c1, o3 = o2 + c2;
  sc->off[255 - 4 * lane] = o0;
  sc->off[254 - 4 * lane] = o1;
  sc->off[253 - 4 * lane] = o2;
  sc->off[252 - 4 * lane] = o3;
  // the bin holding the kc-th key, and the keys in it and above
  const bool here = kc > 0 && o0 < kc && kc <= inc;
  const int d = o1 >= kc ? 255 - 4 * lane : (o2 >= kc ? 254 - 4 * lane : (o3 >= kc ? 253 - 4 * lane : 252 - 4 * lane));
  const int total = o1 >= kc ? o1 : (o2 >= kc ? o2 : (o3 >= kc ? o3 : inc));
  const uint64_t hm = __ballot(here);
  const int src = hm ? __ffsll((long long)hm) - 1 : 0;
  const int cut = hm ? __builtin_amdgcn_readlane(d, src) : 256;
  if (hm && __builtin_amdgcn_readlane(total, src) > LSA_WAVE) return false;
  __builtin_amdgcn_wave_barrier();
  // the candidates at their bins' offsets
#pragma unroll
  for (int m = 0; m < KPL; ++m) {
    if (x[m] != 0 && bin[m] >= cut) sc->cand[sc->off[bin[m]] + atomicAdd(&sc->fill[bin[m]], 1)] = x[m];
  }
  __builtin_amdgcn_wave_barrier();
  // ranks: a candidate's bin offset plus the larger keys of its own bin
  const int nc = cut < 256 ? sc->off[cut] + sc->hist[cut] : 0;
  if (lane < nc) {
    const uint64_t y = sc->cand[lane];
    const int b = bin_of(y);
    const int lo = sc->off[b], hi = lo + sc->hist[b];
    int rank = lo;
    for (int m = lo; m < hi; ++m) rank += sc->cand[m] > y ? 1 : 0;  // nonempty keys are distinct
    if (rank < K) out[rank] = y;
  }
  for (int m = kc + lane; m < kp; m += LSA_WAVE) out[m] = 0;  // EMPTY past the nonempty keys
  return true;
}

// Ranks of up to G placed candidates cand[s0 + q * stride] (q < G; those at or past nc
// skipped): a candidate's rank is its bin's first slot lo_of(b) plus the larger keys among
// the bin's slots [lo_of(b), hi_of(b)); out[rank] = key for ranks below K. Every load is
// unconditional (indexes clamped into the candidates) and the counts branch-free, so the
// G candidates' loads - their keys, their bins' bounds, 4 keys of each bin a round - are
// in flight together. bin_of, lo_of and hi_of must be cheap and unconditional.
template <int G, typename BinOf, typename LoOf, typename HiOf>
__device__ __forceinline__ void rank_candidates(const uint64_t* cand, int nc, int s0, int stride, int K,
                                                uint64_t* out, BinOf bin_of, LoOf lo_of, HiOf hi_of) {
  uint64_t y[G];
  int lo[G], hi[G], rk[G];
#pragma unroll
  for (int q = 0; q < G; ++q) {
    const int s = s0 + q * stride;
    y[q] = cand[s < nc ? s : nc - 1];
  }
  int len = 0;
#pragma unroll
  for (int q = 0; q < G; ++q) {
    const bool on = s0 + q * stride < nc;
    const int b = bin_of(y[q]);
    const int l = lo_of(b), h = hi_of(b);
    lo[q] = on ? l : 0;
    hi[q] = on ? h : 0;
    rk[q] = lo[q];
    len = max(len, hi[q] - lo[q]);
  }
  for (int r0 = 0; r0 < len; r0 += 4) {
#pragma unroll
    for (int q = 0; q < G; ++q) {
      uint64_t v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = cand[min(lo[q] + r0 + u, nc - 1)];
#pragma unroll
      for (int u = 0; u < 4; ++u) rk[q] += (int)(lo[q] + r0 + u < hi[q]) & (int)(v[u] > y[q]);  // live keys are distinct
    }
  }
#pragma unroll
  for (int q = 0; q < G; ++q) {
    if (s0 + q * stride < nc && rk[q] < K) out[rk[q]] = y[q];
  }
}

// The value lane ^ J holds (J a power of two below 64), 32 bits: DPP within a 16-lane row,
// the gfx950 row swaps across rows.
template <int J>
__device__ __forceinline__ uint32_t wave_xor_lane(uint32_t v) {
  if constexpr (J == 1) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);  // quad_perm [1, 0, 3, 2]
  } else if constexpr (J == 2) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);  // quad_perm [2, 3, 0, 1]
  } else if constexpr (J == 4) {
    const int lane = threadIdx.x & (LSA_WAVE - 1);
    const uint32_t up = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x104, 0xF, 0xF, false);  // row_shl:4
    const uint32_t dn = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x114, 0xF, 0xF, false);  // row_shr:4
    return (lane & 4) ? dn : up;
  } else if constexpr (J == 8) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, false);  // row_ror:8
  } else {
    return __builtin_bit_cast(uint32_t, lane_xor(__builtin_bit_cast(float, v), J));
  }
}

// Lanes that keep the smaller value at the step of distance J of a descending bitonic merge
// of blocks of K lanes: those whose lane bits J and K differ.
__host__ __device__ constexpr uint64_t bitonic_min_lanes(int K, int J) {
  uint64_t m = 0;
  for (int l = 0; l < 64; ++l)
    if (((l & J) != 0) != ((l & K) != 0)) m |= 1ull << l;
  return m;
}

// One compare-exchange step of the wave-wide bitonic sort (u64 values as high/low words): a
// lane takes its partner's value when the partner's is larger and the lane keeps maxima, or
// smaller and it keeps minima. One compare and a scalar XOR with a constant lane mask.
template <int K, int J>
__device__ __forceinline__ void wave_bitonic_step(uint32_t& vh, uint32_t& vl) {
  const uint32_t ph = wave_xor_lane<J>(vh), pl = wave_xor_lane<J>(vl);
  const uint64_t v = ((uint64_t)vh << 32) | vl, p = ((uint64_t)ph << 32) | pl;
  constexpr uint64_t kMin = bitonic_min_lanes(K, J);
  const bool take = __builtin_amdgcn_inverse_ballot_w64(__builtin_amdgcn_uicmpl(p, v, 34 /* unsigned > */) ^ kMin);
  vh = take ? ph : vh;
  vl = take ? pl : vl;
}

template <int K>
__device__ __forceinline__ void wave_bitonic_merge(uint32_t& vh, uint32_t& vl) {
  if constexpr (K >= 64) wave_bitonic_step<K, 32>(vh, vl);
  if constexpr (K >= 32) wave_bitonic_step<K, 16>(vh, vl);
  if constexpr (K >= 16) wave_bitonic_step<K, 8>(vh, vl);
  if constexpr (K >= 8) wave_bitonic_step<K, 4>(vh, vl);
  if constexpr (K >= 4) wave_bitonic_step<K, 2>(vh, vl);
  wave_bitonic_step<K, 1>(vh, vl);
}

// The K (<= 32) best of the keys one wave holds in registers (x[m] is key m * LSA_WAVE +
// lane, u-ordered, 0 = EMPTY), sorted descending into out[0..kp) (EMPTY past them), in
// registers: the K-th largest top-16-bit prefix among the lanes' best keys, found bit by bit
// with wave-wide counts, bounds the candidates from below (at least K keys lie at or above
// it, since K lanes each hold one); the candidates are compacted by ballot into cand[0..64)
// and sorted by a 64-lane bitonic sort (21 compare-exchange steps over DPP and row swaps),
// after which lane r holds the r-th best. No LDS atomics, no bins, no score arithmetic:
// the u64 order is the only one used, non-finite scores included. Returns false (every
// lane, before touching out) when more than 64 keys reach the bound; the caller then ranks
// another way. 1 <= K <= 32, kp <= 64.
template <int KPL>
__device__ __forceinline__ bool wave_topk_small(const uint64_t (&x)[KPL], int K, int kp, uint64_t* out,
                                                uint64_t* cand) {
  const int lane = threadIdx.x & (LSA_WAVE - 1);
  uint32_t mh = (uint32_t)(x[0] >> 32);
#pragma unroll
  for (int m = 1; m < KPL; ++m) mh = max(mh, (uint32_t)(x[m] >> 32));
  uint32_t t = 0;
#pragma unroll
  for (int b = 31; b >= 16; --b) {
    const uint32_t c = t | (1u << b);
    if (__popcll(__builtin_amdgcn_uicmp(mh, c, 35 /* unsigned >= */)) >= K) t = c;
  }
  const uint64_t t0 = t ? (uint64_t)t << 32 : 1;  // fewer than K lanes hold keys: every live key
  int nc = 0;
#pragma unroll
  for (int m = 0; m < KPL; ++m) {
    const uint64_t b = __builtin_amdgcn_uicmpl(x[m], t0, 35 /* unsigned >= */);
    const int slot = nc + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0));
    if (__builtin_amdgcn_inverse_ballot_w64(b) && slot < LSA_WAVE) cand[slot] = x[m];
    nc += __popcll(b);
  }
  if (nc > LSA_WAVE) return false;  // uniform
  __builtin_amdgcn_wave_barrier();
  const uint64_t y = lane < nc ? cand[lane] : 0;
  uint32_t vh = (uint32_t)(y >> 32), vl = (uint32_t)y;
  wave_bitonic_merge<2>(vh, vl);
  wave_bitonic_merge<4>(vh, vl);
  wave_bitonic_merge<8>(vh, vl);
  wave_bitonic_merge<16>(vh, vl);
  wave_bitonic_merge<32>(vh, vl);
  wave_bitonic_merge<64>(vh, vl);
  const int kc = nc < K ? nc : K;
  if (lane < kp) out[lane] = lane < kc ? (((uint64_t)vh << 32) | vl) : 0;
  return true;
}

// The K best of the keys one wave holds in registers (x[m] is key m * LSA_WAVE + lane,
// u-ordered, 0 = EMPTY), sorted descending into out[0..kp) (EMPTY past them), for any K:
// the linear score bins of block_topk_hist (256 over [min, max]); every key in the bin of
// the min(K, live)-th key or above is placed at its bin's offset in cand[] (capacity: the
// live keys) and ranked by that offset plus the larger keys of its own bin, read 8 at a
// time. No block barrier: the wave's LDS accesses run in program order and wave_barrier
// keeps the compiler from moving them across the phases. Clears sc->hist and sc->fill
// itself. Returns false (in every lane, before any store) when a score is not finite; the
// caller then takes a block select. `out` and `cand` must not overlap.
template <int KPL>
__device__ __forceinline__ bool wave_topk_sort(const uint64_t (&x)[KPL], int K, int kp, uint64_t* out,
                                               uint64_t* cand, TopkScratch* sc) {
  const int lane = threadIdx.x & (LSA_WAVE - 1);
  float mn = INFINITY, mx = -INFINITY;
  int cnt = 0, bad = 0;
#pragma unroll
  for (int m = 0; m < KPL; ++m) {
    const float s = key_score(x[m]);
    const bool live = x[m] != 0;
    bad |= (live && s - s != 0.0f) ? 1 : 0;  // NaN or infinite
    mn = live ? fminf(mn, s) : mn;
    mx = live ? fmaxf(mx, s) : mx;
    cnt += live ? 1 : 0;
  }
  mn = wave_min(mn);
  mx = wave_max(mx);
  cnt = wave_sum(cnt);
  if (wave_or(bad)) return false;
  const int kc = cnt < K ? cnt : K;
  for (int b = lane; b < 256; b += LSA_WAVE) {
    sc->hist[b] = 0;
    sc->fill[b] = 0;
  }
  const float scale = mx > mn ? 256.0f / (mx - mn) : 0.0f;
  auto bin_of = [&](uint64_t k) {
    const int b = (int)((key_score(k) - mn) * scale);
    return b < 0 ? 0 : (b > 255 ? 255 : b);
  };
  __builtin_amdgcn_wave_barrier();
  int bin[KPL];
#pragma unroll
  for (int m = 0; m < KPL; ++m) {
    bin[m] = bin_of(x[m]);
    if (x[m] != 0) atomicAdd(&sc->hist[bin[m]], 1);
  }
  __builtin_amdgcn_wave_barrier();
  // lane l owns bins 255-4l .. 252-4l; exclusive offsets from the top bin down
  const int c0 = sc->hist[255 - 4 * lane], c1 = sc->hist[254 - 4 * lane];
  const int c2 = sc->hist[253 - 4 * lane], c3 = sc->hist[252 - 4 * lane];
  const int mine = c0 + c1 + c2 + c3;
  const int inc = wave_inclusive_sum(mine);
  const int o0 = inc - mine, o1 = o0 + c0, o2 = o1 + c1, o3 = o2 + c2;
  sc->off[255 - 4 * lane] = o0;
  sc->off[254 - 4 * lane] = o1;
  sc->off[253 - 4 * lane] = o2;
  sc->off[252 - 4 * lane] = o3;
  // the bin holding the kc-th key: it and the bins above are the candidates
  const bool here = kc > 0 && o0 < kc && kc <= inc;
  const int d = o1 >= kc ? 255 - 4 * lane : (o2 >= kc ? 254 - 4 * lane : (o3 >= kc ? 253 - 4 * lane : 252 - 4 * lane));
  const uint64_t hm = __ballot(here);
  const int cut = hm ? __builtin_amdgcn_readlane(d, __ffsll((long long)hm) - 1) : 256;
  __builtin_amdgcn_wave_barrier();
  // the candidates at their bins' offsets: every bin offset and slot claim in flight first
  int off_m[KPL], pos[KPL];
#pragma unroll
  for (int m = 0; m < KPL; ++m) {
    off_m[m] = sc->off[bin[m]];
    pos[m] = x[m] != 0 && bin[m] >= cut ? atomicAdd(&sc->fill[bin[m]], 1) : 0;
  }
#pragma unroll
  for (int m = 0; m < KPL; ++m) {
    if (x[m] != 0 && bin[m] >= cut) cand[off_m[m] + pos[m]] = x[m];
  }
  __builtin_amdgcn_wave_barrier();
  const int nc = cut < 256 ? sc->off[cut] + sc->hist[cut] : 0;
  const auto lo_of = [&](int b) { return sc->off[b]; };
  const auto hi_of = [&](int b) { return sc->off[b] + sc->hist[b]; };
  if (nc <= LSA_WAVE) {  // uniform: one candidate a lane
    if (nc > 0) rank_candidates<1>(cand, nc, lane, LSA_WAVE, K, out, bin_of, lo_of, hi_of);
  } else {
    for (int g0 = 0; g0 < nc; g0 += 4 * LSA_WAVE) rank_candidates<4>(cand, nc, g0 + lane, LSA_WAVE, K, out, bin_of, lo_of, hi_of);
  }
  for (int m = kc + lane; m < kp; m += LSA_WAVE) out[m] = 0;  // EMPTY past the live keys
  return true;
}

// The K best of the block's keys held in registers (x[m] is key m * LSA_BLOCK + tid,
// u-ordered, 0 = EMPTY), sorted descending into out[0..kp) (u == 0 past them), for any K:
// the keys are binned linearly by score over [min, max] into NB bins (a monotone map:
// a higher bin never holds a lower key), the bins' descending offsets found by one block
// scan, and the bin holding the K-th key named; every key in it or above (at most K + 63)
// is placed at its bin's offset in cand[], and its rank is that offset plus the larger keys
// of its own bin. Six barriers, no sort. Returns false (every thread) when a score is not
// finite or a bin holds more than 64 keys (ties, a degenerate spread): the caller falls
// back to a radix select. `out` and `cand` (capacity K + 64) must not overlap. Every
// thread calls it. More bins cost a longer scan and make the bins the ranking reads smaller:
// 2048 bins take ~0.6-0.9 µs off a 4096-key top-1024 against 512.
template <int KPT, int NB>
__device__ __forceinline__ bool topk_bins_regs(const uint64_t (&x)[KPT], int K, int kp, uint64_t* out,
                                               uint64_t* cand, TopkScratch* sc, BinScratchN<NB>* bs) {
  constexpr int BPT = NB / LSA_BLOCK;  // bins a thread owns in the scan
  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1), w = tid / LSA_WAVE;
  float mn = INFINITY, mx = -INFINITY;
  int cnt = 0, bad = 0;
#pragma unroll
  for (int m = 0; m < KPT; ++m) {
    const float sc_ = key_score(x[m]);
    const bool live = x[m] != 0;
    bad |= (live && sc_ - sc_ != 0.0f) ? 1 : 0;  // NaN or infinite
    mn = live ? fminf(mn, sc_) : mn;
    mx = live ? fmaxf(mx, sc_) : mx;
    cnt += live ? 1 : 0;
  }
  for (int b = tid; b < NB; b += LSA_BLOCK) bs->bcnt[b] = 0;
  mn = wave_min(mn);
  mx = wave_max(mx);
  cnt = wave_sum(cnt);
  bad = wave_or(bad);
  if (lane == 0) { sc->wmin[w] = mn; sc->wmax[w] = mx; sc->wcnt[w] = cnt; sc->wbad[w] = bad; }
  __syncthreads();
  mn = fminf(fminf(sc->wmin[0], sc->wmin[1]), fminf(sc->wmin[2], sc->wmin[3]));
  mx = fmaxf(fmaxf(sc->wmax[0], sc->wmax[1]), fmaxf(sc->wmax[2], sc->wmax[3]));
  cnt = sc->wcnt[0] + sc->wcnt[1] + sc->wcnt[2] + sc->wcnt[3];
  bad = sc->wbad[0] | sc->wbad[1] | sc->wbad[2] | sc->wbad[3];
  if (bad) return false;  // uniform: every thread sees the same totals
  const int kc = cnt < K ? cnt : K;
  const float scale = mx > mn ? (float)NB / (mx - mn) : 0.0f;
  auto bin_of = [&](uint64_t k) {
    const int b = (int)((key_score(k) - mn) * scale);
    return b < 0 ? 0 : (b > NB - 1 ? NB - 1 : b);
  };
  int bin[KPT];
#pragma unroll
  for (int m = 0; m < KPT; ++m) {
    bin[m] = bin_of(x[m]);
    if (x[m] != 0) atomicAdd(&bs->bcnt[bin[m]], 1);
  }
  __syncthreads();
  // thread t owns bins NB-1-BPT*t .. NB-BPT*(t+1), from the top: descending exclusive
  // offsets by one block scan; the most crowded bin bounds the in-bin ranking below
  int c[BPT], mine = 0, occ = 0;
#pragma unroll
  for (int e = 0; e < BPT; ++e) {
    c[e] = bs->bcnt[NB - 1 - BPT * tid - e];
    mine += c[e];
    occ = c[e] > occ ? c[e] : occ;
  }
  const int inc = wave_inclusive_sum(mine);
  const int wocc = wave_reduce_bits(occ, 0, [](int a, int b) { return a > b ? a : b; });
  if (lane == LSA_WAVE - 1) bs->wsum[w] = inc;
  if (lane == 0) bs->wocc[w] = wocc;
  __syncthreads();
  int before = 0;
#pragma unroll
  for (int v = 0; v < LSA_WAVES; ++v) before += v < w ? bs->wsum[v] : 0;
  int o = before + inc - mine;
#pragma unroll
  for (int e = 0; e < BPT; ++e) {
    const int b = NB - 1 - BPT * tid - e;
    bs->boff[b] = o;
    if (kc > 0 && o < kc && kc <= o + c[e]) {  // the bin of the kc-th key: one thread
      bs->bcut = b;
      bs->bnc = o + c[e];
    }
    o += c[e];
  }
  if (tid == 0) bs->btot = cnt;
  const int maxocc = max(max(bs->wocc[0], bs->wocc[1]), max(bs->wocc[2], bs->wocc[3]));
  if (kc == 0) {  // nothing live: EMPTY throughout
    for (int m = tid; m < kp; m += LSA_BLOCK) out[m] = 0;
    __syncthreads();
    return true;
  }
  if (maxocc > LSA_WAVE) return false;  // uniform
  __syncthreads();
  const int cut = bs->bcut, nc = bs->bnc;
  // the candidates at their bins' offsets, in cand[]
#pragma unroll
  for (int m = 0; m < KPT; ++m) {
    if (x[m] != 0 && bin[m] >= cut) cand[bs->boff[bin[m]] + atomicSub(&bs->bcnt[bin[m]], 1) - 1] = x[m];
  }
  __syncthreads();
  // ranks: a candidate's bin offset plus the larger keys of its own bin (the bin below
  // starts where this one ends); the bin is read 8 keys at a time, all 8 loads in flight
  // (indexes clamped into the candidates, the ones past the bin masked)
  for (int s = tid; s < nc; s += LSA_BLOCK) {
    const uint64_t y = cand[s];
    const int b = bin_of(y);
    const int lo = bs->boff[b], hi = b > 0 ? bs->boff[b - 1] : bs->btot;
    int rank = lo;
    for (int m0 = lo; m0 < hi; m0 += 8) {
      uint64_t c[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) c[u] = cand[min(m0 + u, nc - 1)];
#pragma unroll
      for (int u = 0; u < 8; ++u) rank += (m0 + u < hi && c[u] > y) ? 1 : 0;  // live keys are distinct
    }
    if (rank < K) out[rank] = y;
  }
  for (int m = kc + tid; m < kp; m += LSA_BLOCK) out[m] = 0;  // EMPTY past the live keys
  __syncthreads();
  return true;
}


// The K best of keys[0..n) (u-ordered, in LDS; n <= KPT * LSA_BLOCK) by topk_bins_regs,
// taking the keys into registers and using keys[] as the candidate buffer (its values are
// gone afterwards). Returns false as topk_bins_regs does (keys[] then untouched).
template <int KPT, int NB>
__device__ __forceinline__ bool block_topk_bins(uint64_t* keys, int n, int K, int kp, uint64_t* out,
                                                TopkScratch* sc, BinScratchN<NB>* bs) {
  uint64_t x[KPT];
#pragma unroll
  for (int m = 0; m < KPT; ++m) {
    const int j = m * LSA_BLOCK + threadIdx.x;
    x[m] = j < n ? keys[j] : 0;
  }
  return topk_bins_regs<KPT, NB>(x, K, kp, out, keys, sc, bs);
}

// The K best of the block's keys held in registers (as topk_bins_regs), sorted descending
// into out[0..kp) by a radix select over the registers (8 passes of 8 bits at most) and a
// bitonic sort of out: the path for any keys, ties and non-finite scores included. 1 <= K.
// Every thread calls it.
template <int KPT>
__device__ __forceinline__ void topk_radix_regs(const uint64_t (&x)[KPT], int K, int kp, uint64_t* out,
                                                RadixState* st) {
  const int tid = threadIdx.x;
  if (tid == 0) { st->prefix = 0; st->mask = 0; st->need = K; st->done = 0; }
  for (int pass = 0; pass < 8; ++pass) {
    const int shift = 56 - 8 * pass;
    st->hist[tid] = 0;  // LSA_BLOCK == 256 bins
    __syncthreads();
    const uint64_t prefix = st->prefix, mask = st->mask;
#pragma unroll
    for (int m = 0; m < KPT; ++m)
      if ((x[m] & mask) == prefix) atomicAdd(&st->hist[(x[m] >> shift) & 255], 1);
    __syncthreads();
    if (tid < LSA_WAVE) {
      const int c0 = st->hist[255 - 4 * tid], c1 = st->hist[254 - 4 * tid];
      const int c2 = st->hist[253 - 4 * tid], c3 = st->hist[252 - 4 * tid];
      const int mine = c0 + c1 + c2 + c3;
      const int inc = wave_inclusive_sum(mine);
      int above = inc - mine;
      const int need = st->need;
      if (above < need && need <= inc) {
        int d = 255 - 4 * tid, c = c0;
        if (above + c0 < need) { above += c0; d -= 1; c = c1;
          if (above + c1 < need) { above += c1; d -= 1; c = c2;
            if (above + c2 < need) { above += c2; d -= 1; c = c3; } } }
        const int rest = need - above;
        st->prefix = prefix | ((uint64_t)d << shift);
        st->mask = mask | (0xFFull << shift);
        st->need = rest;
        st->done = (c == rest) ? 1 : 0;
      }
    }
    __syncthreads();
    if (st->done) break;
  }
  if (tid == 0) st->slot = 0;
  __syncthreads();
  const uint64_t prefix = st->prefix;
  const int done = st->done;
#pragma unroll
  for (int m = 0; m < KPT; ++m) {
    const bool take = done ? (x[m] >= prefix) : (x[m] > prefix);
    if (take) out[atomicAdd(&st->slot, 1)] = x[m];
  }
  __syncthreads();
  if (!done) {
    for (int i = st->slot + tid; i < K; i += LSA_BLOCK) out[i] = prefix;
  }
  for (int j = K + tid; j < kp; j += LSA_BLOCK) out[j] = 0;
  __syncthreads();
  bitonic_sort_desc(out, kp);
}

// The K best of keys[0..n) (u-ordered, in LDS), sorted descending into out[0..kp) with
// u == 0 past K (kp = next_pow2(K)). K <= 64 takes the histogram cut when it leaves at
// most 64 candidates; otherwise a radix select + bitonic sort. 1 <= K <= n. Every thread
// calls it.
__device__ __forceinline__ void block_topk_sorted(const uint64_t* keys, int n, int K, int kp, uint64_t* out,
                                                  TopkScratch* sc, RadixState* st) {
  if (K <= LSA_WAVE && block_topk_hist(keys, n, K, kp, out, sc)) return;
  auto get = [&](int j) -> uint64_t { return keys[j]; };
  radix_select(get, n, K, st);
  radix_collect(get, n, K, st, out);
  for (int j = K + threadIdx.x; j < kp; j += LSA_BLOCK) out[j] = 0;
  __syncthreads();
  bitonic_sort_desc(out, kp);
}

// block_topk_sorted for selects whose K may exceed 64: a larger K over at most 8192 keys
// takes the binned ranking (block_topk_bins, which reuses keys[] as its candidate buffer,
// so the keys are gone afterwards), falling back to the radix select + bitonic sort.
template <int NB>
__device__ __forceinline__ void block_topk_any(uint64_t* keys, int n, int K, int kp, uint64_t* out, TopkScratch* sc,
                                               RadixState* st, BinScratchN<NB>* bs) {
  if (K > LSA_WAVE && n <= 32 * LSA_BLOCK) {
    const bool done = n <= 16 * LSA_BLOCK ? block_topk_bins<16, NB>(keys, n, K, kp, out, sc, bs)
                                          : block_topk_bins<32, NB>(keys, n, K, kp, out, sc, bs);
    if (done) return;
  }
  block_topk_sorted(keys, n, K, kp, out, sc, st);
}

// The K best of keys[0..n) (u-ordered, in LDS), sorted descending into out[0..kp), for a
// select whose levels hold few keys: up to 512 keys are ranked by wave 0 in registers
// (wave_topk_sort, keys[] as its candidate buffer, no block barrier but the one after it);
// up to 4096 by the binned ranking for any K; the histogram / radix selects when those
// decline. keys[] are gone afterwards. flag: one int of LDS. Every thread calls it.
__device__ __forceinline__ void block_topk_fast(uint64_t* keys, int n, int K, int kp, uint64_t* out, TopkScratch* sc,
                                                RadixState* st, BinScratch* bs, int* flag) {
  constexpr int KPL = 8;
  if (n <= KPL * LSA_WAVE) {
    if (threadIdx.x < LSA_WAVE) {
      const int lane = threadIdx.x;
      uint64_t x[KPL];
#pragma unroll
      for (int m = 0; m < KPL; ++m) x[m] = m * LSA_WAVE + lane < n ? keys[m * LSA_WAVE + lane] : 0;
      __builtin_amdgcn_wave_barrier();
      const bool ok = wave_topk_sort<KPL>(x, K, kp, out, keys, sc);
      if (lane == 0) *flag = ok ? 1 : 0;
    }
    __syncthreads();
    if (*flag) return;  // uniform
  }
  if (n <= 16 * LSA_BLOCK && block_topk_bins<16, kTopBins>(keys, n, K, kp, out, sc, bs)) return;
  block_topk_sorted(keys, n, K, kp, out, sc, st);
}

// Closed-form visible count without span ends (reference pipeline.py:184-186).
__device__ __forceinline__ int visible_closed(int64_t position, int rows, int cluster_block, int block_buckets) {
  const int64_t blocks =
      position >= 0 ? position / cluster_block : -((-position + cluster_block - 1) / cluster_block);
  int64_t v = blocks * block_buckets;
  return (int)(v > rows ? rows : v);
}

// Value of tail slot i (after the kept ids) of a read list: the window [window_start,
// position], then the sinks [0, min(sink, window_start)), then -1.
__device__ __forceinline__ int32_t tail_id(int64_t i, int64_t window_start, int64_t n_win, int64_t n_sink) {
  return i < n_win ? (int32_t)(window_start + i) : (i < n_win + n_sink ? (int32_t)(i - n_win) : -1);
}

// Rank-order expansion of one row over span tables (bucket row b holds exactly the ids
// ends[b - 1] .. ends[b] - 1, ends[-1] = 0, in order): pick b keeps the consecutive ids
// [max(begin_b, sink), min(ends[b], window_start)), so the kept list is a concatenation of
// ranges, stored in rank order until top_k, then the window and sink tail, then -1 to
// `width`. The same list expand_walk builds from the member rows, with no member loads.
// Every listed id is stored as map(id) (a paged cache's physical row; the identity without
// a slot table). n_picks <= 64; lds: 129 ints. Every thread of the block calls it; returns
// the length.
__device__ __forceinline__ int expand_spans(const int32_t* picks, int n_picks, const int32_t* ends, int rows,
                                            int64_t position, int window, int sink, int top_k, int32_t* out,
                                            int width, int* lds, SlotRow map = SlotRow{nullptr, 0}) {
  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1), w = tid / LSA_WAVE;
  const int64_t ws = position + 1 - window;
  const int64_t window_start = ws > 0 ? ws : 0;
  if (w == 0) {
    int lo = 0, c = 0;
    const int b = lane < n_picks ? picks[lane] : -1;
    if (b >= 0 && b < rows) {
      const int64_t begin = b > 0 ? ends[b - 1] : 0, end = ends[b];
      const int64_t l = begin > sink ? begin : sink, h = end < window_start ? end : window_start;
      lo = (int)l;
      c = h > l ? (int)(h - l) : 0;
    }
    const int incl = wave_inclusive_sum(c);
    lds[lane] = lo;
    lds[LSA_WAVE + lane] = incl - c;  // first slot of pick `lane`
    if (lane == LSA_WAVE - 1) lds[2 * LSA_WAVE] = incl;
  }
  __syncthreads();
  const int total = lds[2 * LSA_WAVE];
  const int kept = total < top_k ? total : top_k;
  for (int j = w; j < n_picks; j += LSA_WAVES) {  // wave w stores picks w, w + 4, ...
    const int lo = lds[j], p0 = lds[LSA_WAVE + j];
    const int p1 = j + 1 < LSA_WAVE ? lds[LSA_WAVE + j + 1] : total;
    const int e = p1 < kept ? p1 : kept;
    for (int x = p0 + lane; x < e; x += LSA_WAVE) out[x] = map(lo + (x - p0));
  }
  const int64_t n_win = position + 1 - window_start > 0 ? position + 1 - window_start : 0;
  const int64_t n_sink = sink < window_start ? sink : window_start;
  for (int x = kept + tid; x < width; x += LSA_BLOCK) out[x] = map(tail_id(x - kept, window_start, n_win, n_sink));
  return kept + (int)n_win + (int)n_sink;
}

// Writes a list row staged in LDS (`stage`: its first `filled` kept ids, already mapped)
// to `out` in coalesced 16-byte stores: the kept ids, then the tail (window, sinks; mapped
// here), then -1 to `width` (width % 4 == 0, out 16-byte aligned). Every thread calls it
// after the barrier that completes `stage`.
__device__ __forceinline__ void store_staged_row(const int32_t* stage, int filled, int64_t window_start, int64_t n_win,
                                                 int64_t n_sink, int32_t* out, int width, SlotRow map) {
  const int length = filled + (int)n_win + (int)n_sink;
  for (int c = threadIdx.x; c < width / 4; c += LSA_BLOCK) {
    const int s0 = 4 * c;
    int4 v;
    if (s0 + 4 <= filled) {
      v = ((const int4*)stage)[c];
    } else if (s0 >= length) {
      v = make_int4(-1, -1, -1, -1);
    } else {
      int e[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int slot = s0 + k;
        e[k] = slot < filled ? stage[slot] : map(tail_id(slot - filled, window_start, n_win, n_sink));
      }
      v = make_int4(e[0], e[1], e[2], e[3]);
    }
    ((int4*)out)[c] = v;
  }
}

// Rank-order expansion of span tables for any number of picks (expand_spans serves at most
// 64): thread t takes picks [PPT t, PPT (t + 1)), their kept ranges [max(begin, sink),
// min(end, window start)) from the span ends (both ends of every pick in flight at once),
// one block prefix sum places them, every kept id up to top_k goes to its slot of the LDS
// row `stage` (width + 4 ints; 16-byte aligned) mapped, and the row leaves in coalesced
// stores (store_staged_row). Without `stage` (or when width % 4 != 0) the ids are stored
// directly. n_picks <= PPT * LSA_BLOCK; picks in LDS (bucket rows, -1 none). The same list
// as expand_walk. Every thread calls it; returns the length.
template <int PPT>
__device__ __forceinline__ int expand_spans_wide(const int32_t* picks, int n_picks, const int32_t* ends, int rows,
                                                 int64_t position, int window, int sink, int top_k, int32_t* out,
                                                 int width, int32_t* stage, int* scan, SlotRow map) {
  const int tid = threadIdx.x;
  const int64_t ws = position + 1 - window;
  const int64_t window_start = ws > 0 ? ws : 0;
  int32_t eb[PPT], ee[PPT];
  bool ok[PPT];
#pragma unroll
  for (int p = 0; p < PPT; ++p) {  // every pick's two span ends in flight together
    const int j = tid * PPT + p;
    const int b = j < n_picks ? picks[j] : -1;
    ok[p] = b >= 0 && b < rows;
    eb[p] = ends[ok[p] && b > 0 ? b - 1 : 0];
    ee[p] = ends[ok[p] ? b : 0];
  }
  int lo[PPT], cnt[PPT], mine = 0;
#pragma unroll
  for (int p = 0; p < PPT; ++p) {
    const int b = tid * PPT + p < n_picks ? picks[tid * PPT + p] : -1;
    const int64_t begin = b > 0 ? eb[p] : 0;
    const int64_t l = begin > sink ? begin : sink, h = (int64_t)ee[p] < window_start ? ee[p] : window_start;
    lo[p] = (int)l;
    cnt[p] = ok[p] && h > l ? (int)(h - l) : 0;
    mine += cnt[p];
  }
  int total;
  int at = block_exclusive_sum(mine, scan, &total);
  const int kept = total < top_k ? total : top_k;
  const bool staged = stage != nullptr && width % 4 == 0;
  int32_t* dst = staged ? stage : out;
#pragma unroll
  for (int p = 0; p < PPT; ++p) {
    const int e = cnt[p] < kept - at ? cnt[p] : (kept - at > 0 ? kept - at : 0);
    for (int x = 0; x < e; ++x) dst[at + x] = map(lo[p] + x);
    at += cnt[p];
  }
  const int64_t n_win = position + 1 - window_start > 0 ? position + 1 - window_start : 0;
  const int64_t n_sink = sink < window_start ? sink : window_start;
  if (staged) {
    __syncthreads();
    store_staged_row(stage, kept, window_start, n_win, n_sink, out, width, map);
  } else {
    for (int x = kept + tid; x < width; x += LSA_BLOCK) out[x] = map(tail_id(x - kept, window_start, n_win, n_sink));
  }
  return kept + (int)n_win + (int)n_sink;
}

// Rank-order expansion of one row (reference select_fused.py:172-214): picks in rank
// order, member slots in table order, keep ids with sink <= id < window_start until
// top_k are stored; then the window [window_start, position] and the sinks
// [0, min(sink, window_start)). Slots past the length are -1. Returns the length.
// picks lives in LDS (bucket ids, -1 = none). Each thread owns 32 consecutive slots of a
// 8192-slot super-tile, all loaded before one block-wide prefix sum (as 16-byte vectors
// when the cap is a multiple of 32, so a thread's slots lie in one member row; the table
// is then 16-byte aligned). With `stage` (LDS for width + 4 ints, width % 4 == 0, `out`
// 16-byte aligned) the kept ids are scattered into the LDS row without branches and the
// whole row - ids, tail and padding - leaves in coalesced 16-byte stores; without it they
// are stored directly. Listed ids are stored as map(id) (see expand_spans). Every thread of
// the block calls it.
__device__ __forceinline__ int expand_walk(const int32_t* picks, int n_picks, const int32_t* members, int rows,
                                           int cap, int64_t position, int window, int sink, int top_k,
                                           int32_t* out, int width, int* scan, int32_t* stage,
                                           SlotRow map = SlotRow{nullptr, 0}) {
  constexpr int E = 32;
  const int tid = threadIdx.x;
  const int64_t ws = position + 1 - window;
  const int64_t window_start = ws > 0 ? ws : 0;
  const int64_t total_slots = (int64_t)n_picks * cap;
  const bool rowwise = (cap % E) == 0;
  int filled = 0;
  for (int64_t base = 0; base < total_slots && filled < top_k; base += (int64_t)LSA_BLOCK * E) {
    int32_t ids[E];
    const int64_t s0 = base + (int64_t)tid * E;
    if (rowwise) {
      const int32_t b = s0 < total_slots ? picks[s0 / cap] : -1;
      const bool okb = b >= 0 && b < rows;
      const int4* src = (const int4*)(members + (int64_t)(okb ? b : 0) * cap + (okb ? s0 % cap : 0));
#pragma unroll
      for (int v = 0; v < E / 4; ++v) {
        const int4 x = src[v];
        ids[4 * v] = okb ? x.x : -1;
        ids[4 * v + 1] = okb ? x.y : -1;
        ids[4 * v + 2] = okb ? x.z : -1;
        ids[4 * v + 3] = okb ? x.w : -1;
      }
    } else {
      for (int e = 0; e < E; ++e) {
        const int64_t s = s0 + e;
        const int32_t b = s < total_slots ? picks[(int)(s / cap)] : -1;
        const bool okb = b >= 0 && b < rows;
        const int32_t id = members[(int64_t)(okb ? b : 0) * cap + (okb ? (int)(s % cap) : 0)];
        ids[e] = okb ? id : -1;
      }
    }
    uint32_t keep = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const bool ok = (ids[e] >= sink) && ((int64_t)ids[e] < window_start);
      keep |= ok ? (1u << e) : 0u;
    }
    int total;
    const int at = filled + block_exclusive_sum(__popc(keep), scan, &total);
    if (stage) {
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int pos = at + __popc(keep & ((1u << e) - 1u));
        const bool put = ((keep >> e) & 1u) && pos < top_k;
        stage[put ? pos : width] = ids[e];  // slot `width` is a sink for the unkept
      }
    } else {
      int pos = at;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        if ((keep >> e) & 1u) {
          if (pos < top_k) out[pos] = map(ids[e]);
          ++pos;
        }
      }
    }
    filled += total;
  }
  if (filled > top_k) filled = top_k;
  const int64_t n_win = position + 1 - window_start > 0 ? position + 1 - window_start : 0;
  const int64_t n_sink = sink < window_start ? sink : window_start;
  const int length = filled + (int)n_win + (int)n_sink;
  if (stage) {
    __syncthreads();
    for (int c = tid; c < width / 4; c += LSA_BLOCK) {
      const int s0 = 4 * c;
      int4 v;
      if (s0 + 4 <= filled) {
        v = ((const int4*)stage)[c];
      } else if (s0 >= length) {
        v = make_int4(-1, -1, -1, -1);
      } else {
        int e[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int slot = s0 + k;
          e[k] = slot < filled ? stage[slot] : tail_id(slot - filled, window_start, n_win, n_sink);
        }
        v = make_int4(e[0], e[1], e[2], e[3]);
      }
      if (map.row != nullptr) v = make_int4(map(v.x), map(v.y), map(v.z), map(v.w));
      ((int4*)out)[c] = v;
    }
  } else {
    for (int i = tid; i < width - filled; i += LSA_BLOCK)
      out[filled + i] = map(tail_id(i, window_start, n_win, n_sink));
  }
  return length;
}

}  // namespace lsa
