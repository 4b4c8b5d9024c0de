// Bucket-table build on the GPU: contiguous Ward-style segments from the keys.
//
// The index build that precedes the select+read path (the reference builds its bucket tables
// with build_buckets_gpu, pipeline.py:71-116: pooled keys merged by the Ward cost into
// buckets, centroids from the member keys). Here the buckets stay contiguous - every
// bucket is a run of consecutive positions, so a table is its span ends and the decode
// expands a pick from them - and merges adjacent segments only:
//
//   1. pools: the keys of one table (one (batch, kv-head)) cut into pools of `pool`
//      consecutive positions (the last one shorter); a pool's key sum in fp64, positions in
//      order;
//   2. merges: while more than `target` segments remain, the adjacent pair (a, b) with the
//      smallest Ward cost  n_a n_b / (n_a + n_b) * |s_a / n_a - s_b / n_b|^2  merges into
//      one (ties to the leftmost pair; pairs over `max_size` positions never merge);
//   3. out: the segment start positions, [target + 1] per table (the last entry = T).
//
// Every cost is computed in one fixed order of fp64 operations, with no contraction into
// fused multiply-adds: the squared differences d = 0..D-1 fold into 64 partials
// (partial l = sum over k of sq[l + 64 k], k ascending), then halve 32, 16, .., 1 (partial l
// += partial l + h). The merge loop runs in one workgroup per table: costs, sizes and the
// segment links in LDS, the fp64 sums in a global scratch buffer.
#include <float.h>
#include <math.h>

#include "lsa_abi_common.h"
#include "lsa_device.h"

using namespace lsa;

namespace {

constexpr int kPoolThreads = 256;
constexpr int kMergeThreads = 1024;
constexpr int kMergeWaves = kMergeThreads / LSA_WAVE;
constexpr int kMaxPools = 4096;  // LDS-resident segment state (cost, size, links) per table

// fp64 key sum of every (table, pool, dim): positions of the pool in order.
template <typename KT>
__global__ __launch_bounds__(kPoolThreads) void pool_sums_kernel(const KT* keys, int64_t T, int kv_heads, int D,
                                                                 int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                                                                 int pool, int npool, double* sums) {
#pragma clang fp contract(off)
  const int64_t per_table = (int64_t)npool * D;
  const int64_t x = (int64_t)blockIdx.x * kPoolThreads + threadIdx.x;
  const int64_t table = blockIdx.y;
  if (x >= per_table) return;
  const int p = (int)(x / D), d = (int)(x % D);
  const KT* kb = keys + (table / kv_heads) * kv_sb + (table % kv_heads) * kv_sh;
  const int64_t t0 = (int64_t)p * pool;
  const int64_t t1 = t0 + pool < T ? t0 + pool : T;
  double s = 0.0;
  for (int64_t t = t0; t < t1; ++t) s = s + (double)elem<KT>::load(kb, t * kv_st + d);
  sums[table * per_table + x] = s;
}

// Ward cost of adjacent segments a < b (sums at sa / sb, sizes na / nb) on one wave; every
// lane returns it. +inf when the merged segment would exceed max_size.
__device__ double pair_cost(const double* sa, const double* sb, int na, int nb, int D, int max_size) {
#pragma clang fp contract(off)
  if (na + nb > max_size) return INFINITY;
  const int lane = threadIdx.x & (LSA_WAVE - 1);
  const double fa = (double)na, fb = (double)nb;
  double part = 0.0;
  for (int d = lane; d < D; d += LSA_WAVE) {
    const double diff = sa[d] / fa - sb[d] / fb;
    const double sq = diff * diff;
    part = part + sq;
  }
#pragma unroll
  for (int h = LSA_WAVE / 2; h >= 1; h >>= 1) {
    const double other = __shfl_down(part, h, LSA_WAVE);
    if (lane < h) part = part + other;
  }
  const double total = __shfl(part, 0, LSA_WAVE);
  const double w = (fa * fb) / (fa + fb);
  return w * total;
}

// The greedy adjacent merge of one table (one workgroup). Segments are named by their
// first pool; cost[i] is the cost of segment i with the segment after it.
__global__ __launch_bounds__(kMergeThreads) void ward_merge_kernel(double* sums, int64_t T, int D, int pool,
                                                                   int npool, int target, int max_size,
                                                                   int32_t* starts, int32_t* status,
                                                                   int32_t* failed_any) {
  __shared__ double cost[kMaxPools];
  __shared__ int size[kMaxPools];
  __shared__ int nxt[kMaxPools];
  __shared__ int prv[kMaxPools];
  __shared__ double wbest[kMergeWaves];
  __shared__ int wbest_i[kMergeWaves];
  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1), w = tid / LSA_WAVE;
  const int64_t table = blockIdx.x;
  double* ts = sums + table * (int64_t)npool * D;
  for (int i = tid; i < npool; i += kMergeThreads) {
    const int64_t t0 = (int64_t)i * pool;
    size[i] = (int)((t0 + pool < T ? t0 + pool : T) - t0);
    nxt[i] = i + 1 < npool ? i + 1 : -1;
    prv[i] = i - 1;
  }
  __syncthreads();
  for (int i = w; i < npool; i += kMergeWaves) {
    const double c = i + 1 < npool
                         ? pair_cost(ts + (int64_t)i * D, ts + (int64_t)(i + 1) * D, size[i], size[i + 1], D, max_size)
                         : INFINITY;
    if (lane == 0) cost[i] = c;
  }
  __syncthreads();
  int alive = npool;
  int failed = 0;
  while (alive > target) {
    // the leftmost minimum over the segments' costs
    double best = INFINITY;
    int bi = kMaxPools;
    for (int i = tid; i < npool; i += kMergeThreads) {
      const double c = cost[i];
      if (c < best) {
        best = c;
        bi = i;
      }
    }
#pragma unroll
    for (int h = LSA_WAVE / 2; h >= 1; h >>= 1) {
      const double oc = __shfl_xor(best, h, LSA_WAVE);
      const int oi = __shfl_xor(bi, h, LSA_WAVE);
      if (oc < best || (oc == best && oi < bi)) {
        best = oc;
        bi = oi;
      }
    }
    if (lane == 0) {
      wbest[w] = best;
      wbest_i[w] = bi;
    }
    __syncthreads();
    best = wbest[0];
    bi = wbest_i[0];
    for (int k = 1; k < kMergeWaves; ++k) {
      const double oc = wbest[k];
      const int oi = wbest_i[k];
      if (oc < best || (oc == best && oi < bi)) {
        best = oc;
        bi = oi;
      }
    }
    if (!(best < INFINITY)) {  // no pair can merge under max_size
      failed = 1;
      break;
    }
    const int i = bi, j = nxt[i];
    for (int d = tid; d < D; d += kMergeThreads) ts[(int64_t)i * D + d] = ts[(int64_t)i * D + d] + ts[(int64_t)j * D + d];
    __syncthreads();  // every thread has read the links and sums it needs
    if (tid == 0) {
      size[i] += size[j];
      const int k = nxt[j];
      nxt[i] = k;
      if (k >= 0) prv[k] = i;
      cost[j] = INFINITY;
    }
    __syncthreads();
    if (w == 0) {
      const int a = prv[i];
      if (a >= 0) {
        const double c = pair_cost(ts + (int64_t)a * D, ts + (int64_t)i * D, size[a], size[i], D, max_size);
        if (lane == 0) cost[a] = c;
      }
    } else if (w == 1) {
      const int b = nxt[i];
      const double c =
          b >= 0 ? pair_cost(ts + (int64_t)i * D, ts + (int64_t)b * D, size[i], size[b], D, max_size) : INFINITY;
      if (lane == 0) cost[i] = c;
    }
    __syncthreads();
    --alive;
  }
  int32_t* out = starts + table * (int64_t)(target + 1);
  if (failed) {
    // the even cut: valid, increasing positions for every kernel that reads the table later
    for (int r = tid; r < target; r += kMergeThreads) out[r] = (int32_t)((int64_t)r * T / target);
  }
  if (tid == 0) {
    status[table] = failed;
    if (!failed) {
      int p = 0;
      for (int r = 0; r < target; ++r) {
        out[r] = p * pool;
        p = nxt[p];
      }
    } else if (failed_any) {  // system scope: the word may live in pinned host memory
      __hip_atomic_store(failed_any, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    out[target] = (int32_t)T;
  }
}

}  // namespace

extern "C" size_t lsa_ward_segments_scratch_bytes(int64_t tables, int64_t T, int32_t D, int32_t pool) {
  if (tables < 0 || T < 0 || D < 1 || pool < 1) return 0;
  const int64_t npool = (T + pool - 1) / pool;
  return (size_t)(tables * npool * D) * sizeof(double);
}

extern "C" int lsa_ward_segments(const void* keys, int k_dtype, int64_t B, int64_t T, int32_t kv_heads, int32_t D,
                                 int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int32_t pool, int32_t target,
                                 int32_t max_size, void* scratch, size_t scratch_bytes, int32_t* starts,
                                 int32_t* status, int32_t* failed, void* stream) {
  LSA_REQUIRE(keys && scratch && starts && status, LSA_ERR_NULL, "lsa_ward_segments: NULL pointer");
  LSA_REQUIRE(k_dtype == LSA_F32 || k_dtype == LSA_BF16 || k_dtype == LSA_F16, LSA_ERR_DTYPE,
              "lsa_ward_segments: dtype %d", k_dtype);
  LSA_REQUIRE(B >= 1 && T >= 1 && kv_heads >= 1 && D >= 1 && D <= kMergeThreads && pool >= 1 && target >= 1,
              LSA_ERR_SHAPE, "lsa_ward_segments: bad sizes");
  LSA_REQUIRE(T < (1ll << 31), LSA_ERR_SHAPE, "lsa_ward_segments: T = %lld does not fit int32 positions",
              (long long)T);
  const int64_t npool = (T + pool - 1) / pool;
  LSA_REQUIRE(npool <= kMaxPools, LSA_ERR_SHAPE,
              "lsa_ward_segments: %lld pools exceed %d (raise the pool size)", (long long)npool, kMaxPools);
  LSA_REQUIRE(target <= npool, LSA_ERR_SHAPE, "lsa_ward_segments: target %d exceeds the %lld pools", target,
              (long long)npool);
  LSA_REQUIRE(max_size >= pool, LSA_ERR_SHAPE, "lsa_ward_segments: max_size %d below the pool size %d", max_size,
              pool);
  const int64_t tables = B * kv_heads;
  LSA_REQUIRE(tables <= 65535, LSA_ERR_SHAPE, "lsa_ward_segments: too many tables");
  const size_t need = lsa_ward_segments_scratch_bytes(tables, T, D, pool);
  LSA_REQUIRE(scratch_bytes >= need, LSA_ERR_SHAPE, "lsa_ward_segments: scratch %zu bytes, needs %zu", scratch_bytes,
              need);
  hipStream_t s = (hipStream_t)stream;
  double* sums = (double*)scratch;
  const dim3 grid((unsigned)((npool * D + kPoolThreads - 1) / kPoolThreads), (unsigned)tables);
  LSA_DISPATCH_QT(k_dtype, {
    pool_sums_kernel<QT><<<grid, kPoolThreads, 0, s>>>((const QT*)keys, T, kv_heads, D, kv_sb, kv_st, kv_sh, pool,
                                                       (int)npool, sums);
  })
  LSA_LAUNCHED("lsa_ward_segments (pool sums)");
  ward_merge_kernel<<<dim3((unsigned)tables), kMergeThreads, 0, s>>>(sums, T, D, pool, (int)npool, target, max_size,
                                                                     starts, status, failed);
  LSA_LAUNCHED("lsa_ward_segments (merge)");
  return LSA_OK;
}
