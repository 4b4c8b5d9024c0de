// Sparse gather read for gfx950 (reference read_kernel_tiled.py:30-156, read_kernel.py:26-120).
//
// One workgroup (4 wave64) = (query row, kv-head, split). The kv-head's whole query group
// (Hq/Hkv heads) shares every gathered K/V row: a token's row of D elements is read by
// LPT = D/VEC lanes with one 16-byte load each, so a row is fetched once, coalesced, for
// the whole group. A split owns a fixed span of `tiles * NT` list slots; a row with n keys
// has ceil(n / span) active splits and the rest of the grid exits at its first
// instruction, so the grid can be sized from the list width without knowing the lengths.
//
// Latency discipline (decode is a chain of dependent HBM round trips, not a bandwidth
// problem at B=1): every global load is unconditional (invalid slots read row 0 of the
// same cache and are masked to -inf afterwards), so the compiler issues a tile's ids, and
// then all of its K/V rows, before the first wait; the next tile's ids are fetched while
// the current tile computes. Scores are fp32 dot products (scale and log2(e) folded into
// q), the softmax is the online form in the exp2 domain, and the running (m, l, acc) of
// token groups, waves and splits are merged with the usual rescaling. With more than one
// active split each workgroup leaves its partial in the workspace with write-through
// stores; the last to arrive (a per-(row, kv-head) counter, reset by that workgroup)
// loads every partial in one batch and writes the output.
#include <math.h>

#include "lsa_abi_common.h"
#include "lsa_device.h"

using namespace lsa;

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -3.0e38f;  // finite "minus infinity" for the running max
constexpr int kMaxSplits = 256;

// 16 raw bytes of a row -> VEC floats.
template <typename T> struct Row16;
template <> struct Row16<bf16_t> {
  static constexpr int N = 8;
  static __device__ __forceinline__ void cvt(const uint4& u, float* f) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  }
};
template <> struct Row16<_Float16> {
  static constexpr int N = 8;
  static __device__ __forceinline__ void cvt(const uint4& u, float* f) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      _Float16 lo, hi;
      const uint16_t a = (uint16_t)(w[i] & 0xFFFFu), b = (uint16_t)(w[i] >> 16);
      __builtin_memcpy(&lo, &a, 2);
      __builtin_memcpy(&hi, &b, 2);
      f[2 * i] = (float)lo;
      f[2 * i + 1] = (float)hi;
    }
  }
};
template <> struct Row16<float> {
  static constexpr int N = 4;
  static __device__ __forceinline__ void cvt(const uint4& u, float* f) {
    f[0] = __uint_as_float(u.x); f[1] = __uint_as_float(u.y);
    f[2] = __uint_as_float(u.z); f[3] = __uint_as_float(u.w);
  }
};

// Launch geometry of one (dtype, head dim) instance.
// Tiles of 64 tokens: 8 16-byte K/V loads per lane in flight (bf16, D=128). A CU keeps
// only so many misses in flight, so a decode read spreads its tiles over as many CUs as
// possible rather than giving each workgroup more rows.
template <typename T, int D, int GQ>
struct ReadShape {
  static constexpr int VEC = Row16<T>::N;
  static constexpr int LPT = D / VEC;                        // lanes per token row
  static constexpr int TPW = LSA_WAVE / LPT;                 // tokens per wave per load step
  static constexpr int U0 = 64 / (LSA_WAVES * TPW);
  static constexpr int U = U0 < 1 ? 1 : (U0 > 8 ? 8 : U0);   // load steps per tile
  static constexpr int NT = LSA_WAVES * TPW * U;             // tokens per tile
};

struct ReadArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  const int32_t* ids;
  const int32_t* lengths;
  int64_t Tq, Tk;
  int64_t kv_sb, kv_st, kv_sh;  // K/V element strides of batch, token and head
  int Hq, Hkv, W;
  int ids_per_head;
  int chunk;  // > 0: chunked-prefill lists (shared list of the row's chunk + its causal block)
  float scale_log2;
  int empty_nan;
  int span;   // list slots per split (a multiple of the tile)
  int* ws_count;
  float* ws_part;
};

// The keys a (row, kv-head) reads: its own list, or (chunked prefill) its chunk's list
// followed by the chunk's causal block [chunk_start, t].
struct RowList {
  const int32_t* ids;
  int n_list;
  int n;
  int64_t local_start;
};

__device__ __forceinline__ RowList row_list(const ReadArgs& a, int64_t row, int g) {
  RowList r;
  if (a.chunk > 0) {
    const int64_t b = row / a.Tq, t = row % a.Tq;
    const int64_t c = t / a.chunk;
    const int64_t C = (a.Tq + a.chunk - 1) / a.chunk;
    const int64_t li = (b * C + c) * a.Hkv + g;
    int n = a.W > 0 ? a.lengths[li] : 0;
    n = n < 0 ? 0 : (n > a.W ? a.W : n);
    r.ids = a.ids + li * a.W;
    r.n_list = n;
    r.local_start = c * a.chunk;
    r.n = n + (int)(t - c * a.chunk + 1);
  } else {
    const int64_t li = a.ids_per_head ? row * a.Hkv + g : row;
    int n = a.lengths[li];
    n = (n < 0 || a.Tk <= 0) ? 0 : (n > a.W ? a.W : n);
    r.ids = a.ids + li * a.W;
    r.n_list = n;
    r.local_start = 0;
    r.n = n;
  }
  return r;
}

// Token id of list slot j (< hi), or -1; the ids load is unconditional (clamped slot).
__device__ __forceinline__ int32_t slot_id(const RowList& l, int j, int hi) {
  const int jl = j < l.n_list ? j : (l.n_list > 0 ? l.n_list - 1 : 0);
  const int32_t x = l.n_list > 0 ? l.ids[jl] : -1;
  const int32_t local = (int32_t)(l.local_start + (j - l.n_list));
  return j >= hi ? -1 : (j < l.n_list ? x : local);
}

// Split partials cross workgroups that may sit on different XCDs, whose L2s are not
// coherent with each other. They are written and read with system-coherent (write-
// through, cache-bypassing) accesses, so publishing them needs only the stores' own
// completion (s_waitcnt) before the arrival counter - not a device-scope fence, which on
// gfx950 writes back the whole L2.
typedef float f4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void coherent_store(float* p, float x) { *(volatile float*)p = x; }
__device__ __forceinline__ float coherent_load(const float* p) { return *(const volatile float*)p; }
__device__ __forceinline__ float4 coherent_load4(const float* p) {
  const f4v v = *(const volatile f4v*)p;
  return make_float4(v.x, v.y, v.z, v.w);
}

// exp2 on the hardware unit (v_exp_f32): softmax weights that would be denormal flush
// to zero, which the normaliser never notices.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// DPP lane exchange inside a row of 16: dpp_ctrl quad_perm / row mirrors.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// The partner value of lane ^ x for x in {16, 32} (v_permlane16/32_swap on gfx950), else
// a bpermute shuffle.
__device__ __forceinline__ float lane_xor(float v, int x) {
  const int iv = __builtin_bit_cast(int, v);
  const int row = (threadIdx.x & (LSA_WAVE - 1)) >> 4;
  if (x == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(iv, iv, false, false);
    return __builtin_bit_cast(float, (row & 1) ? r[0] : r[1]);
  }
  if (x == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(iv, iv, false, false);
    return __builtin_bit_cast(float, (row & 2) ? r[0] : r[1]);
  }
  return __shfl_xor(v, x, LSA_WAVE);
}

// Sum over each group of N consecutive lanes (N a power of two <= 64), in every lane of
// the group: DPP adds inside rows of 16, lane swaps across rows.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (N >= 2) x += dpp_mov<0xB1>(x);   // quad_perm [1,0,3,2]
  if constexpr (N >= 4) x += dpp_mov<0x4E>(x);   // quad_perm [2,3,0,1]
  if constexpr (N >= 8) x += dpp_mov<0x141>(x);  // row_half_mirror
  if constexpr (N >= 16) x += dpp_mov<0x140>(x); // row_mirror
  if constexpr (N >= 32) x += lane_xor(x, 16);
  if constexpr (N >= 64) x += lane_xor(x, 32);
  return x;
}

// Dot product of 8 packed 16-bit elements (two uint4-halves' worth of words): fp32
// accumulation of exact products (v_dot2c).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
template <typename T>
__device__ __forceinline__ float dot8(const uint32_t* q, const uint4& k) {
  const uint32_t kw[4] = {k.x, k.y, k.z, k.w};
  float p = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (__is_same(T, bf16_t))
      p = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, q[i]), __builtin_bit_cast(bf16x2_t, kw[i]), p,
                                          false);
    else
      p = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, q[i]), __builtin_bit_cast(f16x2_t, kw[i]), p, false);
  }
  return p;
}

template <typename T> __device__ __forceinline__ void store_out(T* p, float x);
template <> __device__ __forceinline__ void store_out<float>(float* p, float x) { *p = x; }
template <> __device__ __forceinline__ void store_out<bf16_t>(bf16_t* p, float x) { p->bits = f32_to_bf16(x); }
template <> __device__ __forceinline__ void store_out<_Float16>(_Float16* p, float x) { *p = (_Float16)x; }

template <typename T, int D, int GQ>
__global__ __launch_bounds__(LSA_BLOCK) void read_kernel(ReadArgs a) {
  using S = ReadShape<T, D, GQ>;
  constexpr int VEC = S::VEC, LPT = S::LPT, TPW = S::TPW, U = S::U, NT = S::NT;
  constexpr int COLS = GQ * D / 4;                       // float4 columns of a partial
  constexpr int RPT = COLS >= LSA_BLOCK ? 1 : LSA_BLOCK / COLS;  // threads per column
  constexpr int CPT = COLS >= LSA_BLOCK ? COLS / LSA_BLOCK : 1;  // columns per thread
  constexpr int PSTRIDE = GQ * (D + 2);                  // floats per partial
  constexpr int BATCH = 16 / CPT;                        // partials loaded per batch
  __shared__ float lds_acc[LSA_WAVES][GQ][D];
  __shared__ float lds_m[LSA_WAVES][GQ];
  __shared__ float lds_l[LSA_WAVES][GQ];
  __shared__ float lds_w[kMaxSplits][GQ];
  __shared__ float lds_pl[kMaxSplits][GQ];
  __shared__ float lds_ltot[GQ];
  __shared__ float4 lds_red[RPT > 1 ? RPT : 1][RPT > 1 ? COLS : 1];
  __shared__ int is_last;

  const int64_t i = blockIdx.x;
  const int s = blockIdx.y;
  const int64_t row = i / a.Hkv;
  const int g = (int)(i % a.Hkv);
  const int tid = threadIdx.x;
  const int lane = tid & (LSA_WAVE - 1);
  const int w = tid / LSA_WAVE;
  const int tg = lane / LPT, lp = lane % LPT;

  const RowList list = row_list(a, row, g);
  const int n_act = (list.n + a.span - 1) / a.span;
  if (s >= (n_act > 0 ? n_act : 1)) return;  // idle split
  T* outp = (T*)a.out + (row * a.Hq + (int64_t)g * GQ) * D;
  if (list.n == 0) {  // nothing to read: zeros (tiled contract) or NaN (v1 contract)
    for (int j = tid; j < GQ * D; j += LSA_BLOCK) store_out<T>(outp + j, a.empty_nan ? NAN : 0.0f);
    return;
  }
  const int lo = s * a.span;
  const int hi = min(lo + a.span, list.n);
  const int64_t b = row / a.Tq;
  const int64_t tstride = a.kv_st;
  const T* kb = (const T*)a.k + b * a.kv_sb + g * a.kv_sh + lp * VEC;
  const T* vb = (const T*)a.v + b * a.kv_sb + g * a.kv_sh + lp * VEC;

  // first tile's ids and the queries go out together
  int32_t id[U];
#pragma unroll
  for (int u = 0; u < U; ++u) id[u] = slot_id(list, lo + (u * LSA_WAVES + w) * TPW + tg, hi);
  // 16-bit rows score with packed dot products on the raw query words (scale applied to
  // the fp32 sum); fp32 rows use FMAs on a pre-scaled query
  constexpr bool PACKED = sizeof(T) == 2;
  uint32_t qw[GQ][4];
  float qf[GQ][VEC];
#pragma unroll
  for (int h = 0; h < GQ; ++h) {
    const uint4 raw = *(const uint4*)((const T*)a.q + (row * a.Hq + (int64_t)g * GQ + h) * D + lp * VEC);
    qw[h][0] = raw.x; qw[h][1] = raw.y; qw[h][2] = raw.z; qw[h][3] = raw.w;
    if constexpr (!PACKED) {
      Row16<T>::cvt(raw, qf[h]);
#pragma unroll
      for (int e = 0; e < VEC; ++e) qf[h][e] *= a.scale_log2;
    }
  }
  float m[GQ], l[GQ], acc[GQ][VEC];
#pragma unroll
  for (int h = 0; h < GQ; ++h) {
    m[h] = kNegBig;
    l[h] = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[h][e] = 0.0f;
  }

  for (int base = lo; base < hi; base += NT) {
    // all K/V rows of the tile in flight at once
    bool ok[U];
    uint4 kr[U], vr[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ok[u] = id[u] >= 0 && id[u] < a.Tk;
      const uint64_t off = (uint64_t)(uint32_t)(ok[u] ? id[u] : 0) * (uint32_t)tstride;
      kr[u] = *(const uint4*)(kb + off);
      vr[u] = *(const uint4*)(vb + off);
    }
    // next tile's ids while this one computes
    const int nb = base + NT;
#pragma unroll
    for (int u = 0; u < U; ++u) id[u] = slot_id(list, nb + (u * LSA_WAVES + w) * TPW + tg, hi);

    float sc[GQ][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int h = 0; h < GQ; ++h) {
        float p;
        if constexpr (PACKED) {
          p = dot8<T>(qw[h], kr[u]);
        } else {
          float kf[VEC];
          Row16<T>::cvt(kr[u], kf);
          p = 0.0f;
#pragma unroll
          for (int e = 0; e < VEC; ++e) p = fmaf(qf[h][e], kf[e], p);
        }
        p = group_sum<LPT>(p);
        if constexpr (PACKED) p *= a.scale_log2;
        sc[h][u] = ok[u] ? p : -INFINITY;
      }
    }
    const bool rescale = base != lo;  // the first tile starts from an empty state
#pragma unroll
    for (int h = 0; h < GQ; ++h) {
      float mt = m[h];
#pragma unroll
      for (int u = 0; u < U; ++u) mt = fmaxf(mt, sc[h][u]);
      if (rescale) {
        const float alpha = fast_exp2(m[h] - mt);
        l[h] *= alpha;
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[h][e] *= alpha;
      }
      m[h] = mt;
#pragma unroll
      for (int u = 0; u < U; ++u) sc[h][u] = fast_exp2(sc[h][u] - mt);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float vf[VEC];
      Row16<T>::cvt(vr[u], vf);
#pragma unroll
      for (int h = 0; h < GQ; ++h) {
        l[h] += sc[h][u];
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[h][e] = fmaf(sc[h][u], vf[e], acc[h][e]);
      }
    }
  }

  // merge the token groups of the wave (lanes that hold the same dims)
#pragma unroll
  for (int x = LPT; x < LSA_WAVE; x <<= 1) {
#pragma unroll
    for (int h = 0; h < GQ; ++h) {
      const float mo = lane_xor(m[h], x);
      const float lo_ = lane_xor(l[h], x);
      const float mn = fmaxf(m[h], mo);
      const float a1 = fast_exp2(m[h] - mn), a2 = fast_exp2(mo - mn);
      l[h] = l[h] * a1 + lo_ * a2;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float ao = lane_xor(acc[h][e], x);
        acc[h][e] = acc[h][e] * a1 + ao * a2;
      }
      m[h] = mn;
    }
  }
  if (tg == 0) {
#pragma unroll
    for (int h = 0; h < GQ; ++h) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) lds_acc[w][h][lp * VEC + e] = acc[h][e];
      if (lp == 0) { lds_m[w][h] = m[h]; lds_l[w][h] = l[h]; }
    }
  }
  __syncthreads();

  // merge the waves: thread j owns (head, dim) pairs j, j + 256, ...
  float* part = n_act > 1 ? a.ws_part + (i * (int64_t)gridDim.y + s) * PSTRIDE : nullptr;
  for (int j = tid; j < GQ * D; j += LSA_BLOCK) {
    const int h = j / D, d = j % D;
    float M = kNegBig;
#pragma unroll
    for (int ww = 0; ww < LSA_WAVES; ++ww) M = fmaxf(M, lds_m[ww][h]);
    float L = 0.0f, A = 0.0f;
#pragma unroll
    for (int ww = 0; ww < LSA_WAVES; ++ww) {
      const float f = fast_exp2(lds_m[ww][h] - M);
      L += lds_l[ww][h] * f;
      A += lds_acc[ww][h][d] * f;
    }
    if (n_act == 1) {
      store_out<T>(outp + j, L > 0.0f ? A / L : (a.empty_nan ? NAN : 0.0f));
    } else {
      coherent_store(part + 2 * GQ + j, A);
      if (d == 0) { coherent_store(part + h, M); coherent_store(part + GQ + h, L); }
    }
  }
  if (n_act == 1) return;

  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
  __syncthreads();
  if (tid == 0)
    is_last = __hip_atomic_fetch_add(&a.ws_count[i], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n_act - 1;
  __syncthreads();
  if (!is_last) return;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  // every active split has arrived: reset the counter for the next launch
  if (tid == 0) __hip_atomic_store(&a.ws_count[i], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // combine: the first batch of accumulator columns and every (m, l) are loaded together
  const float* parts = a.ws_part + i * (int64_t)gridDim.y * PSTRIDE;
  const int r = tid / COLS % RPT;
  float4 first[CPT][BATCH];
#pragma unroll
  for (int cc = 0; cc < CPT; ++cc) {
    const int c = (tid % COLS) + cc * LSA_BLOCK;
#pragma unroll
    for (int bb = 0; bb < BATCH; ++bb) {
      const int sp = r + bb * RPT;
      const int sl = sp < n_act ? sp : 0;
      first[cc][bb] = coherent_load4(parts + (int64_t)sl * PSTRIDE + 2 * GQ + 4 * c);
    }
  }
  for (int t = tid; t < n_act * GQ; t += LSA_BLOCK) {
    const int sp = t / GQ, h = t % GQ;
    const float* ps = parts + (int64_t)sp * PSTRIDE;
    const float pm = coherent_load(ps + h), pl = coherent_load(ps + GQ + h);
    lds_w[sp][h] = pm;
    lds_pl[sp][h] = pl;
  }
  __syncthreads();
  // per-head maximum and normaliser: wave w reduces heads w, w + 4, ... with the splits
  // strided over its lanes (a fixed reduction order, so the output is deterministic)
  for (int h = w; h < GQ; h += LSA_WAVES) {
    float M = kNegBig;
    for (int sp = lane; sp < n_act; sp += LSA_WAVE) M = fmaxf(M, lds_w[sp][h]);
#pragma unroll
    for (int x = LSA_WAVE / 2; x >= 1; x >>= 1) M = fmaxf(M, __shfl_xor(M, x, LSA_WAVE));
    float L = 0.0f;
    for (int sp = lane; sp < n_act; sp += LSA_WAVE) {
      const float f = fast_exp2(lds_w[sp][h] - M);
      L += lds_pl[sp][h] * f;
      lds_w[sp][h] = f;
    }
#pragma unroll
    for (int x = LSA_WAVE / 2; x >= 1; x >>= 1) L += __shfl_xor(L, x, LSA_WAVE);
    if (lane == 0) lds_ltot[h] = L;
  }
  __syncthreads();
#pragma unroll
  for (int cc = 0; cc < CPT; ++cc) {
    const int c = (tid % COLS) + cc * LSA_BLOCK;
    const int h = (4 * c) / D;
    float4 sum = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int bb = 0; bb < BATCH; ++bb) {
      const int sp = r + bb * RPT;
      const float f = sp < n_act ? lds_w[sp][h] : 0.0f;
      sum.x += f * first[cc][bb].x; sum.y += f * first[cc][bb].y;
      sum.z += f * first[cc][bb].z; sum.w += f * first[cc][bb].w;
    }
    for (int sb = BATCH * RPT; sb < n_act; sb += BATCH * RPT) {  // more splits than one batch
      float4 x[BATCH];
#pragma unroll
      for (int bb = 0; bb < BATCH; ++bb) {
        const int sp = r + sb + bb * RPT;
        x[bb] = coherent_load4(parts + (int64_t)(sp < n_act ? sp : 0) * PSTRIDE + 2 * GQ + 4 * c);
      }
#pragma unroll
      for (int bb = 0; bb < BATCH; ++bb) {
        const int sp = r + sb + bb * RPT;
        const float f = sp < n_act ? lds_w[sp][h] : 0.0f;
        sum.x += f * x[bb].x; sum.y += f * x[bb].y; sum.z += f * x[bb].z; sum.w += f * x[bb].w;
      }
    }
    if (RPT > 1) {
      lds_red[r][c] = sum;
    } else {
      const float L = lds_ltot[h];
      const float inv = L > 0.0f ? 1.0f / L : 0.0f;
      const float e = a.empty_nan ? NAN : 0.0f;
      store_out<T>(outp + 4 * c + 0, L > 0.0f ? sum.x * inv : e);
      store_out<T>(outp + 4 * c + 1, L > 0.0f ? sum.y * inv : e);
      store_out<T>(outp + 4 * c + 2, L > 0.0f ? sum.z * inv : e);
      store_out<T>(outp + 4 * c + 3, L > 0.0f ? sum.w * inv : e);
    }
  }
  if (RPT > 1) {
    __syncthreads();
    for (int c = tid; c < COLS; c += LSA_BLOCK) {
      float4 sum = lds_red[0][c];
#pragma unroll
      for (int rr = 1; rr < RPT; ++rr) {
        const float4 x = lds_red[rr][c];
        sum.x += x.x; sum.y += x.y; sum.z += x.z; sum.w += x.w;
      }
      const int h = (4 * c) / D;
      const float L = lds_ltot[h];
      const float inv = L > 0.0f ? 1.0f / L : 0.0f;
      const float e = a.empty_nan ? NAN : 0.0f;
      store_out<T>(outp + 4 * c + 0, L > 0.0f ? sum.x * inv : e);
      store_out<T>(outp + 4 * c + 1, L > 0.0f ? sum.y * inv : e);
      store_out<T>(outp + 4 * c + 2, L > 0.0f ? sum.z * inv : e);
      store_out<T>(outp + 4 * c + 3, L > 0.0f ? sum.w * inv : e);
    }
  }
}

template <typename T, int D>
void launch_read_gq(const ReadArgs& a, int gq, dim3 grid, hipStream_t s) {
  switch (gq) {
    case 1: read_kernel<T, D, 1><<<grid, LSA_BLOCK, 0, s>>>(a); break;
    case 2: read_kernel<T, D, 2><<<grid, LSA_BLOCK, 0, s>>>(a); break;
    case 4: read_kernel<T, D, 4><<<grid, LSA_BLOCK, 0, s>>>(a); break;
    default: read_kernel<T, D, 8><<<grid, LSA_BLOCK, 0, s>>>(a); break;
  }
}

template <typename T>
void launch_read(const ReadArgs& a, int D, int gq, dim3 grid, hipStream_t s) {
  switch (D) {
    case 32: launch_read_gq<T, 32>(a, gq, grid, s); break;
    case 64: launch_read_gq<T, 64>(a, gq, grid, s); break;
    case 128: launch_read_gq<T, 128>(a, gq, grid, s); break;
    default: launch_read_gq<T, 256>(a, gq, grid, s); break;
  }
}

template <typename T, int GQ>
int tile_of(int D) {
  switch (D) {
    case 32: return ReadShape<T, 32, GQ>::NT;
    case 64: return ReadShape<T, 64, GQ>::NT;
    case 128: return ReadShape<T, 128, GQ>::NT;
    default: return ReadShape<T, 256, GQ>::NT;
  }
}

int tile_tokens(int dtype, int D, int gq) {
  // fp16 rows have the bf16 geometry; only the group of 8 changes the tile
  if (dtype == LSA_F32) return gq > 4 ? tile_of<float, 8>(D) : tile_of<float, 4>(D);
  return gq > 4 ? tile_of<bf16_t, 8>(D) : tile_of<bf16_t, 4>(D);
}

// Slots per split: whole tiles, enough that `splits` of them cover the width.
int split_span(int dtype, int D, int gq, int W, int splits) {
  const int nt = tile_tokens(dtype, D, gq);
  const int tiles = (W + nt - 1) / nt;
  const int per = (tiles + splits - 1) / splits;
  return (per > 0 ? per : 1) * nt;
}

int check_read_common(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t Tq, int64_t Tk,
                      int32_t Hq, int32_t Hkv, int32_t D, int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                      const int32_t* ids, const int32_t* lengths, int32_t W, const void* out) {
  LSA_REQUIRE(q && k && v && ids && lengths && out, LSA_ERR_NULL, "sparse read: NULL pointer");
  LSA_REQUIRE(dtype == LSA_F32 || dtype == LSA_BF16 || dtype == LSA_F16, LSA_ERR_DTYPE, "sparse read: dtype %d",
              dtype);
  LSA_REQUIRE(D == 32 || D == 64 || D == 128 || D == 256, LSA_ERR_SHAPE, "sparse read: head dim %d not in {32,64,128,256}",
              D);
  LSA_REQUIRE(Hq >= 1 && Hkv >= 1 && Hq % Hkv == 0, LSA_ERR_SHAPE, "sparse read: Hq %d must group onto Hkv %d", Hq,
              Hkv);
  const int gq = Hq / Hkv;
  LSA_REQUIRE(gq == 1 || gq == 2 || gq == 4 || gq == 8, LSA_ERR_SHAPE, "sparse read: group size %d not in {1,2,4,8}",
              gq);
  LSA_REQUIRE(B >= 0 && Tq >= 0 && Tk >= 0 && W >= 0, LSA_ERR_SHAPE, "sparse read: negative size");
  LSA_REQUIRE(Tk <= 0x7FFFFFFF, LSA_ERR_SHAPE, "sparse read: Tk too large for int32 ids");
  const uintptr_t mis = ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) & 15;
  LSA_REQUIRE(mis == 0, LSA_ERR_ALIGN, "sparse read: q/k/v must be 16-byte aligned");
  const int64_t esize = dtype == LSA_F32 ? 4 : 2;
  LSA_REQUIRE(kv_sb >= 0 && kv_st >= D && kv_sh >= D, LSA_ERR_SHAPE,
              "sparse read: K/V strides (%lld, %lld, %lld) must leave rows of %d elements apart", (long long)kv_sb,
              (long long)kv_st, (long long)kv_sh, D);
  LSA_REQUIRE(((kv_sb | kv_st | kv_sh) * esize) % 16 == 0, LSA_ERR_ALIGN,
              "sparse read: K/V strides must keep rows 16-byte aligned");
  return LSA_OK;
}

}  // namespace

extern "C" int32_t lsa_read_tile_tokens(int dtype, int32_t D, int32_t group) {
  if (!(D == 32 || D == 64 || D == 128 || D == 256) || group < 1) return 0;
  return tile_tokens(dtype, D, group);
}

extern "C" size_t lsa_read_scratch_bytes(int64_t rows, int32_t Hq, int32_t Hkv, int32_t D, int32_t splits) {
  if (splits <= 1 || rows <= 0 || Hkv <= 0 || Hq <= 0) return 0;
  const int64_t n = rows * Hkv;
  const int64_t gq = Hq / Hkv;
  return (size_t)n * splits * (size_t)(gq * (D + 2)) * sizeof(float);
}

extern "C" int lsa_read(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t Tq, int64_t Tk,
                        int32_t Hq, int32_t Hkv, int32_t D, int64_t kv_batch_stride, int64_t kv_token_stride,
                        int64_t kv_head_stride, const int32_t* ids, const int32_t* lengths, int32_t W,
                        int ids_per_head, float scale, int empty_nan, int32_t splits, int32_t* counters,
                        void* scratch, size_t scratch_bytes, void* out, void* stream) {
  int rc = check_read_common(q, k, v, dtype, B, Tq, Tk, Hq, Hkv, D, kv_batch_stride, kv_token_stride,
                             kv_head_stride, ids, lengths, W, out);
  if (rc != LSA_OK) return rc;
  LSA_REQUIRE(splits >= 1 && splits <= kMaxSplits, LSA_ERR_SHAPE, "lsa_read: splits in [1, %d], got %d", kMaxSplits,
              splits);
  const int64_t rows = B * Tq;
  LSA_REQUIRE(rows * Hkv <= 0x7FFFFFFF, LSA_ERR_SHAPE, "lsa_read: too many rows");
  const size_t need = lsa_read_scratch_bytes(rows, Hq, Hkv, D, splits);
  LSA_REQUIRE(need == 0 || (scratch && counters && scratch_bytes >= need), LSA_ERR_WORKSPACE,
              "lsa_read: counters/scratch missing or scratch %zu < %zu bytes", scratch_bytes, need);
  if (rows * Hkv == 0) return LSA_OK;
  ReadArgs a;
  a.q = q; a.k = k; a.v = v; a.out = out; a.ids = ids; a.lengths = lengths;
  a.Tq = Tq; a.Tk = Tk; a.Hq = Hq; a.Hkv = Hkv; a.W = W; a.ids_per_head = ids_per_head ? 1 : 0; a.chunk = 0;
  a.kv_sb = kv_batch_stride; a.kv_st = kv_token_stride; a.kv_sh = kv_head_stride;
  a.scale_log2 = scale * kLog2e; a.empty_nan = empty_nan ? 1 : 0;
  a.span = split_span(dtype, D, Hq / Hkv, W, splits);
  a.ws_count = counters;
  a.ws_part = need ? (float*)scratch : nullptr;
  const dim3 grid((unsigned)(rows * Hkv), (unsigned)splits);
  hipStream_t s = (hipStream_t)stream;
  const int gq = Hq / Hkv;
  if (dtype == LSA_BF16) launch_read<bf16_t>(a, D, gq, grid, s);
  else if (dtype == LSA_F16) launch_read<_Float16>(a, D, gq, grid, s);
  else launch_read<float>(a, D, gq, grid, s);
  LSA_LAUNCHED("lsa_read");
  return LSA_OK;
}

extern "C" int lsa_read_chunked(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t T,
                                int64_t Tk, int32_t Hq, int32_t Hkv, int32_t D, int64_t kv_batch_stride,
                                int64_t kv_token_stride, int64_t kv_head_stride, const int32_t* ids,
                                const int32_t* lengths, int32_t W, int32_t chunk, float scale, void* out,
                                void* stream) {
  int rc = check_read_common(q, k, v, dtype, B, T, Tk, Hq, Hkv, D, kv_batch_stride, kv_token_stride,
                             kv_head_stride, ids, lengths, W, out);
  if (rc != LSA_OK) return rc;
  LSA_REQUIRE(chunk >= 1, LSA_ERR_SHAPE, "lsa_read_chunked: chunk must be >= 1");
  LSA_REQUIRE(T <= Tk, LSA_ERR_SHAPE, "lsa_read_chunked: %lld query rows exceed the cache %lld", (long long)T,
              (long long)Tk);
  LSA_REQUIRE(B * T * Hkv <= 0x7FFFFFFF, LSA_ERR_SHAPE, "lsa_read_chunked: too many rows");
  if (B * T * Hkv == 0) return LSA_OK;
  ReadArgs a;
  a.q = q; a.k = k; a.v = v; a.out = out; a.ids = ids; a.lengths = lengths;
  a.Tq = T; a.Tk = Tk; a.Hq = Hq; a.Hkv = Hkv; a.W = W; a.ids_per_head = 1; a.chunk = chunk;
  a.kv_sb = kv_batch_stride; a.kv_st = kv_token_stride; a.kv_sh = kv_head_stride;
  a.scale_log2 = scale * kLog2e; a.empty_nan = 0;
  a.span = split_span(dtype, D, Hq / Hkv, W + chunk, 1);  // one split covers the whole row
  a.ws_count = nullptr; a.ws_part = nullptr;
  const dim3 grid((unsigned)(B * T * Hkv), 1u);
  hipStream_t s = (hipStream_t)stream;
  const int gq = Hq / Hkv;
  if (dtype == LSA_BF16) launch_read<bf16_t>(a, D, gq, grid, s);
  else if (dtype == LSA_F16) launch_read<_Float16>(a, D, gq, grid, s);
  else launch_read<float>(a, D, gq, grid, s);
  LSA_LAUNCHED("lsa_read_chunked");
  return LSA_OK;
}
