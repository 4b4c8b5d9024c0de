// Device side of the fused decode step: arguments, LDS layouts, the select and reader
// roles and the kernel, plus the per-element-type launcher that each decode_<type>.hip
// instantiates (one translation unit per type, compiled in parallel).
#pragma once

#include <math.h>

#include "lsa_abi_common.h"
#include "lsa_read_dev.h"
#include "lsa_select_dev.h"

namespace lsa {
namespace decode {

constexpr int kMaxPicks = LSA_WAVE;  // the record of a unit is polled by one wave
constexpr int kMaxReaders = 256;     // readers per unit (split partials of the combine)
constexpr int kRecordCopies = 8;     // copies of every record, polled by different readers
constexpr size_t kMaxLds = 64 * 1024;

// Phase hooks: no-ops unless a build defines DECODE_MARK(k) (timestamps for profiling).
#ifndef DECODE_MARK
#define DECODE_MARK(k) ((void)0)
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
  int64_t row_tables, group_tables;
  const int32_t* positions;
  int cluster_block, block_buckets;
  int K, kp, window, sink, top_k, W;
  int S, cs;           // select splits and columns per split
  int span, NR;        // slots per read part, readers per unit
  float scale_log2;
  int spin_limit;
  int skip_publish;    // test hook: select workgroups never publish the record (readers give up)
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
  int pick[kMaxPicks], start[kMaxPicks], n[kMaxPicks], abase[kMaxPicks];
  int wcnt[LSA_WAVES];
  int filled, pparts, bad;
};

constexpr size_t sel_keys_offset() { return (sizeof(SelLds) + 15) & ~(size_t)15; }
template <int D, int GQ>
constexpr size_t rd_ids_offset() {
  return (sizeof(RdLds<D, GQ>) + 15) & ~(size_t)15;
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

template <typename T, typename CT, int D, int GQ>
__device__ __forceinline__ void select_role(const DecodeArgs& a, char* smem, int64_t i, int s) {
  constexpr int SPAN = D / 16;
  constexpr bool BF16_MODE = __is_same(CT, bf16_t);
  SelLds& sh = *(SelLds*)smem;
  uint64_t* keys = (uint64_t*)(smem + sel_keys_offset());  // [rows]
  uint64_t* best = keys + a.rows;                           // [kp]
  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1), w = tid / LSA_WAVE;
  const int64_t r = i / a.G;
  const int g = (int)(i % a.G);
  const int64_t position = a.positions[r];
  const int64_t t = r * a.row_tables + g * a.group_tables;
  const CT* cent = (const CT*)a.centroids + t * a.rows * (int64_t)D;
  const int32_t* ends = a.ends ? a.ends + t * a.rows : nullptr;
  const int c0 = s * a.cs;
  const int c1 = min(c0 + a.cs, a.rows);
  const int n_local = c1 > c0 ? c1 - c0 : 0;
  const int vis = ends ? 0 : visible_closed(position, a.rows, a.cluster_block, a.block_buckets);
  const int64_t lim = position + 1;
  DECODE_MARK(0);

  float qs[SPAN];
  group_mean_slice<T, SPAN, GQ>((const T*)a.q + (r * a.Hq + (int64_t)g * GQ) * D, tid & 15, BF16_MODE, qs);
  score_keys<CT, SPAN>(
      qs, cent, D, n_local, [&](int j) { return c0 + j; },
      [&](int j) { return ends ? (int64_t)ends[c0 + j] <= lim : c0 + j < vis; }, keys + c0);
  DECODE_MARK(1);

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

  // kept members of every pick (sink <= id < window start). Span tables: the range
  // [ends[b - 1], ends[b]) clipped to [sink, window start), from two ends words. Otherwise
  // wave w counts picks w, w + 4, ... eight at a time; a member row streams through the
  // wave in 16-byte lane loads (256 slots per wave load; 64 four-byte loads without
  // vec_rows), counted with ballots
  const int32_t* tab = a.members + t * (int64_t)a.rows * a.cap;
  const int64_t wstart = window_start_of(position, a.window);
  constexpr int MJ = 8;
  if (a.spans) {
    if (w == 0 && lane < a.K) {
      const int b = sh.pick[lane];
      const int64_t begin = b > 0 ? ends[b - 1] : 0, end = b >= 0 ? ends[b] : 0;
      const int64_t lo = begin > a.sink ? begin : a.sink, hi = end < wstart ? end : wstart;
      sh.cnt[lane] = b >= 0 && hi > lo ? (int)(hi - lo) : 0;
      sh.first[lane] = (int)lo;
    }
  }
  for (int jb = 0; jb < (a.spans ? 0 : a.K); jb += MJ * LSA_WAVES) {
    int cnt[MJ];
    int b[MJ];
#pragma unroll
    for (int m = 0; m < MJ; ++m) {
      const int j = jb + m * LSA_WAVES + w;
      b[m] = j < a.K ? sh.pick[j] : -1;
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
        if (j < a.K) sh.cnt[j] = cnt[m];
      }
    }
  }
  __syncthreads();
  DECODE_MARK(5);
  if (w == 0) {
    const int c = lane < a.K ? sh.cnt[lane] : 0;
    int incl = c;
#pragma unroll
    for (int d = 1; d < LSA_WAVE; d <<= 1) {
      const int y = __shfl_up(incl, d, LSA_WAVE);
      if (lane >= d) incl += y;
    }
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

template <typename T, int D, int GQ>
__device__ __forceinline__ void reader_role(const DecodeArgs& a, char* smem, int64_t i, int role) {
  using S = ReadShape<T, D, GQ>;
  constexpr int VEC = S::VEC, LPT = S::LPT;
  constexpr int PSTRIDE = GQ * (D + 2);
  RdLds<D, GQ>& sh = *(RdLds<D, GQ>*)smem;
  int32_t* ids = (int32_t*)(smem + rd_ids_offset<D, GQ>());  // [span]
  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1), w = tid / LSA_WAVE;
  const int K = a.K, span = a.span, words = 2 * K;
  const int64_t r = i / a.G;
  const int g = (int)(i % a.G);
  const int64_t position = a.positions[r];
  const int64_t wstart = window_start_of(position, a.window);
  const int64_t n_win = position + 1 - wstart > 0 ? position + 1 - wstart : 0;
  const int64_t n_sink = a.sink < wstart ? a.sink : wstart;
  const int n_tail = (int)(n_win + n_sink);
  const int32_t* mine = a.record + (role % kRecordCopies) * a.cstride + i * words;
  DECODE_MARK(0);

  // the query rows go out before the wait
  const T* qrow = (const T*)a.q + (r * a.Hq + (int64_t)g * GQ) * D;
  QueryRegs<T, D, GQ> qr;
  qr.load(qrow, a.scale_log2);

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
    int prev = __shfl_up(end, 1, LSA_WAVE);
    if (lane == 0) prev = 0;
    const int n = lane < K ? end - prev : 0;
    const int parts = (n + span - 1) / span;
    int incl = parts;
#pragma unroll
    for (int d = 1; d < LSA_WAVE; d <<= 1) {
      const int y = __shfl_up(incl, d, LSA_WAVE);
      if (lane >= d) incl += y;
    }
    if (lane < K) {
      sh.pick[lane] = wa - 2;
      sh.start[lane] = prev;
      sh.n[lane] = n;
      sh.abase[lane] = incl - parts;
    }
    const int filled = __shfl(end, K - 1, LSA_WAVE);
    const int pparts = __shfl(incl, K - 1, LSA_WAVE);
    if (lane == 0) {
      sh.filled = filled;
      sh.pparts = pparts;
      sh.bad = bad;
      if (bad && a.status) __hip_atomic_store(a.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
  __syncthreads();
  DECODE_MARK(1);
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

  const int filled = sh.filled, pparts = sh.pparts;
  const int n_act = pparts + (n_tail + span - 1) / span;  // dense parts: picks' then the tail's
  const int n_part = n_act < a.NR ? n_act : a.NR;        // readers with work (one partial each)
  int32_t* lrow = a.lists + i * (int64_t)a.W;
  const int32_t* tab = a.members + (r * a.row_tables + g * a.group_tables) * (int64_t)a.rows * a.cap;
  const int lp = lane % LPT;
  const T* kb = (const T*)a.k + r * a.kv_sb + g * a.kv_sh + lp * VEC;
  const T* vb = (const T*)a.v + r * a.kv_sb + g * a.kv_sh + lp * VEC;
  AttnState<T, D, GQ> st;
  st.clear();
  bool fresh = true;
  for (int p = role; p < n_act; p += a.NR) {
    int n, slot0;
    if (p < pparts) {
      // pick j holds dense parts [abase[j], abase[j] + parts_j): the last pick whose base
      // is <= p (bases are nondecreasing; picks without parts share the next one's base)
      const uint64_t le = __ballot(lane < K && sh.abase[lane < K ? lane : 0] <= p);
      const int j = (int)__popcll(le) - 1;
      const int u = p - sh.abase[j];
      const int lo_rank = u * span;
      n = min(span, sh.n[j] - lo_rank);
      slot0 = sh.start[j] + lo_rank;
      if (a.spans) {  // the kept members are consecutive ids from the record's first one
        const int32_t first = sh.pick[j] + lo_rank;
        for (int k = tid; k < n; k += LSA_BLOCK) {
          ids[k] = first + k;
          lrow[slot0 + k] = first + k;
        }
        __syncthreads();
      } else {
        // ranks [lo_rank, lo_rank + n) of the pick's kept members, in table order
        const int32_t* row = tab + (int64_t)sh.pick[j] * a.cap;
        const uint64_t below = (1ull << lane) - 1ull;
        for (int c0 = 0, run = 0; c0 < a.cap && run < lo_rank + n; c0 += LSA_BLOCK) {
          const int e = c0 + tid;
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
          if (keep && rank >= 0 && rank < n) {
            ids[rank] = id;
            lrow[slot0 + rank] = id;
          }
          run += tot;
          __syncthreads();  // wcnt is rewritten by the next chunk; ids are complete
        }
      }
    } else {
      const int t0 = (p - pparts) * span;
      n = min(span, n_tail - t0);
      slot0 = filled + t0;
      for (int k = tid; k < n; k += LSA_BLOCK) {
        const int32_t id = tail_id(t0 + k, wstart, n_win, n_sink);
        ids[k] = id;
        lrow[slot0 + k] = id;
      }
      __syncthreads();
    }
    DECODE_MARK(2);
    attend_tiles<T, D, GQ>(
        qr, kb, vb, a.kv_st, a.Tk, 0, n,
        [&](int jj) {
          const int32_t x = ids[jj < n ? jj : 0];
          return jj < n ? x : -1;
        },
        a.scale_log2, fresh, st);
    fresh = false;
    __syncthreads();  // ids are rewritten by the next part
    DECODE_MARK(3);
  }
  // the list's padding [length, W) is shared out over the unit's readers
  {
    const int length = filled + n_tail;
    const int per = (a.W - length + a.NR - 1) / a.NR;
    const int p0 = length + role * per;
    const int p1 = min(p0 + per, a.W);
    for (int k = p0 + tid; k < p1; k += LSA_BLOCK) lrow[k] = -1;
  }

  T* outp = (T*)a.out + (r * a.Hq + (int64_t)g * GQ) * D;
  float* parts = a.ws_part + i * (int64_t)a.NR * PSTRIDE;
  if (role < n_part) {
    merge_token_groups<T, D, GQ>(st);
    finish_span<T, D, GQ>(sh.rd, st, n_part == 1, outp, n_part > 1 ? parts + (int64_t)role * PSTRIDE : nullptr, 0);
  }
  DECODE_MARK(4);
  if (!arrive_last(&a.rd_count[i], a.NR, &sh.rd.flag)) return;
  DECODE_MARK(5);
  if (n_part > 1) {
    combine_partials<T, D, GQ>(sh.rd, parts, n_part, outp, 0);
  } else if (n_part == 0) {  // nothing to read: zeros
    for (int k = tid; k < GQ * D; k += LSA_BLOCK) store_out<T>(outp + k, 0.0f);
  }
  for (int x = tid; x < kRecordCopies * words; x += LSA_BLOCK) {
    const int c = x / words, k = x - c * words;
    coherent_store_i32(a.record + c * a.cstride + i * words + k, 0);
  }
  DECODE_MARK(6);
}

template <typename T, typename CT, int D, int GQ>
__global__ __launch_bounds__(LSA_BLOCK) void decode_flat_kernel(DecodeArgs a) {
  extern __shared__ __align__(16) char smem[];
  const int64_t units = a.R * a.G;
  const int64_t id = blockIdx.x;
  const int64_t nsel = units * a.S;
  if (id < nsel) {
    select_role<T, CT, D, GQ>(a, smem, id % units, (int)(id / units));
  } else {
    const int64_t rid = id - nsel;  // readers: unit fastest, then role (low roles have work)
    reader_role<T, D, GQ>(a, smem, rid % units, (int)(rid / units));
  }
}

// ------------------------------------------------------------------ launch

template <typename T, typename CT, int D>
void launch_gq(const DecodeArgs& a, int gq, dim3 grid, size_t shmem, hipStream_t s) {
  switch (gq) {
    case 1: decode_flat_kernel<T, CT, D, 1><<<grid, LSA_BLOCK, shmem, s>>>(a); break;
    case 2: decode_flat_kernel<T, CT, D, 2><<<grid, LSA_BLOCK, shmem, s>>>(a); break;
    case 4: decode_flat_kernel<T, CT, D, 4><<<grid, LSA_BLOCK, shmem, s>>>(a); break;
    default: decode_flat_kernel<T, CT, D, 8><<<grid, LSA_BLOCK, shmem, s>>>(a); break;
  }
}

template <typename T, typename CT>
void launch_d(const DecodeArgs& a, int D, int gq, dim3 grid, size_t shmem, hipStream_t s) {
  switch (D) {
    case 32: launch_gq<T, CT, 32>(a, gq, grid, shmem, s); break;
    case 64: launch_gq<T, CT, 64>(a, gq, grid, shmem, s); break;
    case 128: launch_gq<T, CT, 128>(a, gq, grid, shmem, s); break;
    default: launch_gq<T, CT, 256>(a, gq, grid, shmem, s); break;
  }
}

template <typename T>
void launch_type(const DecodeArgs& a, bool bf16_table, int D, int gq, dim3 grid, size_t shmem, hipStream_t s) {
  if (bf16_table) launch_d<T, bf16_t>(a, D, gq, grid, shmem, s);
  else launch_d<T, float>(a, D, gq, grid, shmem, s);
}

// Defined by decode_bf16.hip, decode_f16.hip and decode_f32.hip.
void launch_bf16(const DecodeArgs& a, bool bf16_table, int D, int gq, dim3 grid, size_t shmem, hipStream_t s);
void launch_f16(const DecodeArgs& a, bool bf16_table, int D, int gq, dim3 grid, size_t shmem, hipStream_t s);
void launch_f32(const DecodeArgs& a, bool bf16_table, int D, int gq, dim3 grid, size_t shmem, hipStream_t s);

}  // namespace decode
}  // namespace lsa
