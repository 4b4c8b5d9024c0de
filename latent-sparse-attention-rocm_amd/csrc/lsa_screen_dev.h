// The canonical top-K of a set of bucket rows, found on the matrix cores with the exact
// result: a bf16 MFMA screen with a proven error bound, then the canonical (fp64-ordered)
// score of only the rows that can still reach the top-K. Shared by every select that
// scores a whole table in one workgroup (the batched decode's select workgroups, the
// standalone fused select and its prefill use, the tree select's two levels, and the
// replicated decode readers).
//
//  1. screen: every visible row is scored with bf16 16x16x32 MFMAs (fp32 sums) together
//     with S_r = sum_d |q_d| |c_rd| (the same MFMA on the absolute values). Products of
//     bf16 operands are exact in fp32, so any fp32 summation order of the D products lies
//     within 127 * 2^-23 * S_r < 2^-16 S_r of the exact dot product, and the canonical
//     score (fp64 sums, one fp32 rounding) within 2^-24 |exact| + 2^-48 S_r <= 2^-23 S_r of
//     it: |screen - canonical| < 2^-15 S_r. Each row gets the interval [lo, hi] = screen
//     -/+ (2^-14 S_r + 2^-90), which holds its canonical score.
//  2. cut: at least K rows have lo >= L for any L up to the K-th largest lo, so the
//     canonical K-th best score is >= L and every row of the canonical top-K has hi >= L.
//     L is the lower edge of a 256-bin histogram of lo; the candidates are the rows whose
//     hi falls in that bin or above (a superset of hi >= L: the bin map is monotone).
//  3. the candidates (usually K plus a few) get the canonical score and one wave ranks
//     their packed keys; the best K are the canonical top-K, ties to the lower bucket.
// Non-finite screens or more than 64 candidates take the exact path for every row.
#pragma once

#include "lsa_read_dev.h"
#include "lsa_select_dev.h"

namespace lsa {

constexpr int kScreenMaxRows = 1024;
constexpr int kScreenMaxCand = LSA_WAVE;

struct ScreenLds {
  float lo[kScreenMaxRows];  // screen - bound (-inf: not a visible candidate); the exact path's u64 keys
  float hi[kScreenMaxRows];  // screen + bound
  int hist[256];
  uint64_t ckey[kScreenMaxCand];
  int cand[kScreenMaxCand];
  float wmin[LSA_WAVES], wmax[LSA_WAVES];
  int wcnt[LSA_WAVES], wbad[LSA_WAVES];
  int ncand, cut;
  TopkScratch tks;
  RadixState st;
};

// True when screen_topk serves a table: bf16 scoring, head dim 32/64/128, at most
// kScreenMaxRows rows and 64 picks.
__host__ __device__ inline bool screen_fits(int D, int rows, int K) {
  return (D == 32 || D == 64 || D == 128) && rows <= kScreenMaxRows && K >= 1 && K <= LSA_WAVE;
}

// Whether the screen pays: up to kScreenMinRows rows the exact scoring takes one round
// trip of centroid loads (256 rows of 16-bit operands in flight a workgroup), while the
// screen takes two (the rows, then the candidates' re-score). Measured on the tree
// decode's selects (128 nodes, then <= 256 candidates): 20.5 us exact vs 22.8 us
// screened; on the 32k prefill select's 512-row tables the screen wins (102 vs 123 us).
constexpr int kScreenMinRows = 256;
__host__ __device__ inline bool screen_pays(int D, int rows, int K) {
  return rows > kScreenMinRows && screen_fits(D, rows, K);
}

// The screen's B operand from the bf16-rounded query slice `qs` (16-lane layout: lane p
// holds dims SPAN p .. SPAN p + SPAN): lane (row4 = lane / 16, col = lane % 16) holds dims
// 32 c + 8 row4 .. + 8 of column col; column 0 = the query, column 1 = its absolute
// values, the rest zero. Every lane of the wave calls it (shuffles).
template <int D>
__device__ __forceinline__ void screen_operand(const float* qs, uint4* bq) {
  constexpr int SPAN = D / 16;
  const int lane = threadIdx.x & (LSA_WAVE - 1), row4 = lane >> 4, col = lane & 15;
  uint32_t qpk[SPAN / 2];
#pragma unroll
  for (int k = 0; k < SPAN / 2; ++k)
    qpk[k] = (uint32_t)f32_to_bf16(qs[2 * k]) | ((uint32_t)f32_to_bf16(qs[2 * k + 1]) << 16);
#pragma unroll
  for (int c = 0; c < D / 32; ++c) {
    uint32_t v4[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int d = 32 * c + 8 * row4 + 2 * k;  // first of the two dims of word k
      const uint32_t x = (uint32_t)__shfl((int)qpk[(2 * k % SPAN) / 2], d / SPAN, LSA_WAVE);
      v4[k] = col == 0 ? x : (col == 1 ? (x & 0x7FFF7FFFu) : 0u);
    }
    bq[c] = make_uint4(v4[0], v4[1], v4[2], v4[3]);
  }
}

// The K best candidates j < n (table row row_of(j) >= 0 of `cent`, kept when vis_of(j)),
// sorted descending as u-ordered packed keys into out[0..kp) (0 past the K-th), the column
// of a key being its row. qs: the bf16-rounded query slice (16-lane layout). GB: 16-row
// groups a wave has in flight per round trip. row_of and vis_of may load from memory (their
// loads go out with the centroid rows). n <= kScreenMaxRows, 1 <= K <= 64, kp =
// next_pow2(K). Every thread calls it; `out` is complete after a barrier (included).
template <int D, int GB, typename RowOf, typename VisOf>
__device__ __forceinline__ void screen_topk(const float* qs, const bf16_t* cent, int n, RowOf row_of, VisOf vis_of,
                                            int K, int kp, uint64_t* out, ScreenLds& ex) {
  constexpr int NM = D / 32;    // 32-dim chunks of a centroid row (MFMA K)
  constexpr int SPAN = D / 16;
  constexpr float kBound = 6.103515625e-05f;       // 2^-14
  constexpr float kTiny = 8.077935669463161e-28f;  // 2^-90
  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1), w = tid / LSA_WAVE;
  const int row4 = lane >> 4, col = lane & 15;
  uint4 bq[NM];
  screen_operand<D>(qs, bq);
  ex.hist[tid] = 0;  // LSA_BLOCK == 256 bins
  if (tid == 0) ex.ncand = 0;

  // 1. screen: wave w takes 16-row groups w, w + 4, ...; GB groups' rows in flight at once
  int bad = 0;
  const int ngrp = (n + 15) / 16;
  for (int gb = w; gb < ngrp; gb += LSA_WAVES * GB) {
    uint4 A[GB][NM];
    bool vis[GB][4];
    int rr[GB][4];
#pragma unroll
    for (int gi = 0; gi < GB; ++gi) {
      const int grp = gb + LSA_WAVES * gi;
      const int jm = min(16 * grp + col, n - 1);
      const int rm = row_of(jm);
      const int m = rm >= 0 ? rm : 0;
#pragma unroll
      for (int c = 0; c < NM; ++c) A[gi][c] = *(const uint4*)(cent + (int64_t)m * D + 32 * c + 8 * row4);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int j = min(16 * grp + 4 * row4 + u, n - 1);
        rr[gi][u] = row_of(j);
        vis[gi][u] = rr[gi][u] >= 0 && vis_of(j);
      }
    }
#pragma unroll
    for (int gi = 0; gi < GB; ++gi) {
      const int grp = gb + LSA_WAVES * gi;
      if (grp >= ngrp) break;  // wave-uniform
      f32x4_t cs = {0.0f, 0.0f, 0.0f, 0.0f}, cb = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < NM; ++c) {
        cs = Mfma16<bf16_t>::run(A[gi][c], bq[c], cs);
        const uint4 ab = make_uint4(A[gi][c].x & 0x7FFF7FFFu, A[gi][c].y & 0x7FFF7FFFu, A[gi][c].z & 0x7FFF7FFFu,
                                    A[gi][c].w & 0x7FFF7FFFu);
        cb = Mfma16<bf16_t>::run(ab, bq[c], cb);
      }
      // lane (row4, 0) holds the screens of candidates 16 grp + 4 row4 + u, lane (row4, 1)
      // their S
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float sabs = __shfl(cb[u], (lane + 1) & (LSA_WAVE - 1), LSA_WAVE);
        const int j = 16 * grp + 4 * row4 + u;
        if (col == 0 && j < n) {
          const float s = cs[u];
          const float bnd = sabs * kBound + kTiny;
          const bool fin = (s - s == 0.0f) && (bnd - bnd == 0.0f);
          bad |= (vis[gi][u] && !fin) ? 1 : 0;
          ex.lo[j] = vis[gi][u] ? s - bnd : -INFINITY;
          ex.hi[j] = vis[gi][u] ? s + bnd : -INFINITY;
        }
      }
    }
  }
  __syncthreads();

  // 2. visible count, range of lo, histogram cut
  float mn = INFINITY, mx = -INFINITY;
  int cnt = 0;
  for (int j = tid; j < n; j += LSA_BLOCK) {
    const float x = ex.lo[j];
    const bool live = x != -INFINITY;
    mn = live ? fminf(mn, x) : mn;
    mx = live ? fmaxf(mx, x) : mx;
    cnt += live ? 1 : 0;
  }
  mn = wave_min(mn);
  mx = wave_max(mx);
  cnt = wave_sum(cnt);
  bad = wave_or(bad);
  if (lane == 0) { ex.wmin[w] = mn; ex.wmax[w] = mx; ex.wcnt[w] = cnt; ex.wbad[w] = bad; }
  __syncthreads();
  mn = fminf(fminf(ex.wmin[0], ex.wmin[1]), fminf(ex.wmin[2], ex.wmin[3]));
  mx = fmaxf(fmaxf(ex.wmax[0], ex.wmax[1]), fmaxf(ex.wmax[2], ex.wmax[3]));
  cnt = ex.wcnt[0] + ex.wcnt[1] + ex.wcnt[2] + ex.wcnt[3];
  bool slow = (ex.wbad[0] | ex.wbad[1] | ex.wbad[2] | ex.wbad[3]) != 0;  // uniform
  const float scale = mx > mn ? 256.0f / (mx - mn) : 0.0f;
  auto bin_of = [&](float x) {
    const float b = (x - mn) * scale;
    return b < 0.0f ? 0 : (b >= 255.0f ? 255 : (int)b);
  };
  int cut = 0;  // cnt <= K: every visible row is a candidate
  if (!slow && cnt > K) {
    for (int j = tid; j < n; j += LSA_BLOCK) {
      const float x = ex.lo[j];
      if (x != -INFINITY) atomicAdd(&ex.hist[bin_of(x)], 1);
    }
    __syncthreads();
    if (w == 0) {
      // lane l owns bins 255 - 4l .. 252 - 4l; the highest bin whose suffix count reaches K
      const int c0 = ex.hist[255 - 4 * lane], c1 = ex.hist[254 - 4 * lane];
      const int c2 = ex.hist[253 - 4 * lane], c3 = ex.hist[252 - 4 * lane];
      const int mine = c0 + c1 + c2 + c3;
      const int inc = wave_inclusive_sum(mine);
      const int above = inc - mine;
      const bool here = above < K && K <= inc;
      const int d = above + c0 >= K ? 255 - 4 * lane
                  : (above + c0 + c1 >= K ? 254 - 4 * lane : (above + c0 + c1 + c2 >= K ? 253 - 4 * lane
                                                                                         : 252 - 4 * lane));
      const uint64_t hm = __ballot(here);
      const int cutv = __shfl(d, hm ? __ffsll((long long)hm) - 1 : 0, LSA_WAVE);
      if (lane == 0) ex.cut = cutv;
    }
    __syncthreads();
    cut = ex.cut;
  }
  if (!slow) {
    const uint64_t below = (1ull << lane) - 1ull;
    for (int j0 = w * LSA_WAVE; j0 < n; j0 += LSA_BLOCK) {  // one LDS atomic a wave and pass
      const int j = j0 + lane;
      const float x = j < n ? ex.hi[j] : -INFINITY;
      const bool take = x != -INFINITY && (cnt <= K || bin_of(x) >= cut);
      const uint64_t m = __ballot(take);
      if (m == 0) continue;  // wave-uniform
      int base = 0;
      if (lane == 0) base = atomicAdd(&ex.ncand, (int)__popcll(m));
      base = __builtin_amdgcn_readfirstlane(base);
      const int slot = base + (int)__popcll(m & below);
      if (take && slot < kScreenMaxCand) ex.cand[slot] = j;
    }
    __syncthreads();
    slow = ex.ncand > kScreenMaxCand;
  }

  if (!slow) {
    // 3. canonical scores of the candidates (16 lanes a row, 16 rows a pass); one wave
    // ranks their keys
    const int nc = ex.ncand;
    for (int jb = 0; jb < nc; jb += LSA_BLOCK / 16) {
      const int jj = jb + (tid >> 4);
      const int j = ex.cand[jj < nc ? jj : 0];
      const int m = row_of(j);
      SpanRaw<bf16_t, SPAN> raw;
      raw.load(cent + (int64_t)m * D + (tid & 15) * SPAN);
      double acc = 0.0;
#pragma unroll
      for (int e = 0; e < SPAN; ++e) acc = fma((double)qs[e], (double)raw.at(e), acc);
      const float sc = score_tree16(acc);
      if ((tid & 15) == 0 && jj < nc) ex.ckey[jj] = key_to_u(pack_key(sc, m));
    }
    __syncthreads();
    if (w == 0) {
      // each candidate's rank among the nc keys (read back from LDS, a broadcast a step; a
      // tie goes to the lower slot), then the K best in rank order, zeros up to kp
      const uint64_t v = lane < nc ? ex.ckey[lane] : 0;
      int rank = 0;
      for (int j = 0; j < nc; ++j) {
        const uint64_t o = ex.ckey[j];
        rank += (o > v || (o == v && j < lane)) ? 1 : 0;
      }
      if (lane < nc && rank < kp) out[rank] = rank < K ? v : 0;
      if (lane >= nc && lane < kp) out[lane] = 0;
    }
  } else {
    // the canonical score of every visible candidate, then the block top-K
    uint64_t* keys = (uint64_t*)ex.lo;  // lo and hi: kScreenMaxRows u64
    score_keys<bf16_t, SPAN>(qs, cent, D, n, row_of, [&](int j) { return vis_of(j); }, keys);
    __syncthreads();
    block_topk_sorted(keys, n, K, kp, out, &ex.tks, &ex.st);
  }
  __syncthreads();
}

}  // namespace lsa
