// Sparse gather read for gfx950 (reference read_kernel_tiled.py:30-156, read_kernel.py:26-120).
//
// One workgroup = (query row, kv-head, split). The kv-head's query group (Hq/Hkv heads)
// shares every gathered K/V row: a token's row of D elements is read by LPT = D/VEC
// lanes with one 16-byte load each (VEC elements), so each K or V row is fetched once,
// coalesced, for the whole GQA group. A tile's ids and all of its K/V loads are issued
// before any arithmetic (one memory round trip per tile). Scores are fp32 dot products
// (scale and log2(e) folded into q), softmax is the online form in the exp2 domain, and
// the running state (m, l, acc) of the token groups, waves and splits is merged with the
// usual rescaling. With splits > 1 each workgroup leaves its partial in the workspace and
// the last one to arrive (a per-(row, kv-head) counter) combines them and resets the
// counter for the next launch.
#include <math.h>

#include "lsa_abi_common.h"
#include "lsa_device.h"

using namespace lsa;

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -3.0e38f;  // finite "minus infinity" for the running max

template <typename T> struct Vec16;
template <> struct Vec16<bf16_t> {
  static constexpr int N = 8;
  static __device__ __forceinline__ void load(const bf16_t* p, float* f) {
    const uint4 u = *(const uint4*)p;
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  }
};
template <> struct Vec16<_Float16> {
  static constexpr int N = 8;
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ void load(const _Float16* p, float* f) {
    const h8 h = *(const h8*)p;
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)h[i];
  }
};
template <> struct Vec16<float> {
  static constexpr int N = 4;
  static __device__ __forceinline__ void load(const float* p, float* f) {
    const float4 u = *(const float4*)p;
    f[0] = u.x; f[1] = u.y; f[2] = u.z; f[3] = u.w;
  }
};

struct ReadArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  const int32_t* ids;
  const int32_t* lengths;
  int64_t Tq, Tk;
  int Hq, Hkv, W;
  int ids_per_head;
  int chunk;  // > 0: chunked-prefill lists (shared list of the row's chunk + its causal block)
  float scale_log2;
  int empty_nan;
  int S;
  int* ws_count;
  float* ws_part;
};

// The keys a (row, kv-head) reads: either its own list, or (chunked prefill) its chunk's
// list followed by the chunk's causal block [chunk_start, t].
struct RowList {
  const int32_t* ids;
  int n_list;
  int n;
  int64_t local_start;
  __device__ __forceinline__ int32_t id(int j) const {
    return j < n_list ? ids[j] : (int32_t)(local_start + (j - n_list));
  }
};

__device__ __forceinline__ RowList row_list(const ReadArgs& a, int64_t row, int g) {
  RowList r;
  if (a.chunk > 0) {
    const int64_t b = row / a.Tq, t = row % a.Tq;
    const int64_t c = t / a.chunk;
    const int64_t C = (a.Tq + a.chunk - 1) / a.chunk;
    const int64_t li = (b * C + c) * a.Hkv + g;
    int n = a.lengths[li];
    n = n < 0 ? 0 : (n > a.W ? a.W : n);
    r.ids = a.ids + li * a.W;
    r.n_list = n;
    r.local_start = c * a.chunk;
    r.n = n + (int)(t - c * a.chunk + 1);
  } else {
    const int64_t li = a.ids_per_head ? row * a.Hkv + g : row;
    int n = a.lengths[li];
    n = n < 0 ? 0 : (n > a.W ? a.W : n);
    r.ids = a.ids + li * a.W;
    r.n_list = n;
    r.local_start = 0;
    r.n = n;
  }
  return r;
}

template <typename T> __device__ __forceinline__ void store_out(T* p, float x);
template <> __device__ __forceinline__ void store_out<float>(float* p, float x) { *p = x; }
template <> __device__ __forceinline__ void store_out<bf16_t>(bf16_t* p, float x) { p->bits = f32_to_bf16(x); }
template <> __device__ __forceinline__ void store_out<_Float16>(_Float16* p, float x) { *p = (_Float16)x; }

template <typename T, int D, int GQ>
__global__ __launch_bounds__(LSA_BLOCK) void read_kernel(ReadArgs a) {
  using V = Vec16<T>;
  constexpr int VEC = V::N;
  constexpr int LPT = D / VEC;          // lanes per token row
  constexpr int TPW = LSA_WAVE / LPT;   // tokens per wave per step
  constexpr int U = 4;                  // steps per tile (loads in flight per lane: 2U)
  constexpr int NT = LSA_WAVES * TPW * U;
  __shared__ float lds_acc[LSA_WAVES][GQ][D];
  __shared__ float lds_m[LSA_WAVES][GQ];
  __shared__ float lds_l[LSA_WAVES][GQ];
  __shared__ int is_last;

  const int64_t i = blockIdx.x;
  const int s = blockIdx.y;
  const int64_t row = i / a.Hkv;
  const int g = (int)(i % a.Hkv);
  const int lane = threadIdx.x & (LSA_WAVE - 1);
  const int w = threadIdx.x / LSA_WAVE;
  const int tg = lane / LPT, lp = lane % LPT;

  const RowList list = row_list(a, row, g);
  const int per = (list.n + a.S - 1) / a.S;
  const int lo = s * per;
  const int hi = min(lo + per, list.n);
  const int64_t b = row / a.Tq;
  const int64_t tstride = (int64_t)a.Hkv * D;
  const T* kb = (const T*)a.k + (b * a.Tk * a.Hkv + g) * (int64_t)D + lp * VEC;
  const T* vb = (const T*)a.v + (b * a.Tk * a.Hkv + g) * (int64_t)D + lp * VEC;

  float qf[GQ][VEC];
#pragma unroll
  for (int h = 0; h < GQ; ++h) {
    V::load((const T*)a.q + (row * a.Hq + (int64_t)g * GQ + h) * D + lp * VEC, qf[h]);
#pragma unroll
    for (int e = 0; e < VEC; ++e) qf[h][e] *= a.scale_log2;
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
    int32_t id[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int slot = base + (u * LSA_WAVES + w) * TPW + tg;
      int32_t x = slot < hi ? list.id(slot) : -1;
      id[u] = (x >= 0 && x < a.Tk) ? x : -1;
    }
    float kf[U][VEC], vf[U][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (id[u] >= 0) {
        V::load(kb + id[u] * tstride, kf[u]);
        V::load(vb + id[u] * tstride, vf[u]);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) { kf[u][e] = 0.0f; vf[u][e] = 0.0f; }
      }
    }
#pragma unroll
    for (int h = 0; h < GQ; ++h) {
      float sc[U];
      float mt = kNegBig;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float p = 0.0f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) p = fmaf(qf[h][e], kf[u][e], p);
#pragma unroll
        for (int x = LPT / 2; x >= 1; x >>= 1) p += __shfl_xor(p, x, LSA_WAVE);
        sc[u] = id[u] >= 0 ? p : -INFINITY;
        mt = fmaxf(mt, sc[u]);
      }
      const float mn = fmaxf(m[h], mt);
      const float alpha = exp2f(m[h] - mn);
      l[h] *= alpha;
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[h][e] *= alpha;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float pu = exp2f(sc[u] - mn);
        l[h] += pu;
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[h][e] = fmaf(pu, vf[u][e], acc[h][e]);
      }
      m[h] = mn;
    }
  }

  // merge the token groups of the wave (lanes that hold the same dims)
#pragma unroll
  for (int x = LPT; x < LSA_WAVE; x <<= 1) {
#pragma unroll
    for (int h = 0; h < GQ; ++h) {
      const float mo = __shfl_xor(m[h], x, LSA_WAVE);
      const float lo_ = __shfl_xor(l[h], x, LSA_WAVE);
      const float mn = fmaxf(m[h], mo);
      const float a1 = exp2f(m[h] - mn), a2 = exp2f(mo - mn);
      l[h] = l[h] * a1 + lo_ * a2;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float ao = __shfl_xor(acc[h][e], x, LSA_WAVE);
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
  float* part = a.S > 1 ? a.ws_part + (i * a.S + s) * (int64_t)(GQ * (D + 2)) : nullptr;
  for (int j = threadIdx.x; j < GQ * D; j += LSA_BLOCK) {
    const int h = j / D, d = j % D;
    float M = kNegBig;
#pragma unroll
    for (int ww = 0; ww < LSA_WAVES; ++ww) M = fmaxf(M, lds_m[ww][h]);
    float L = 0.0f, A = 0.0f;
#pragma unroll
    for (int ww = 0; ww < LSA_WAVES; ++ww) {
      const float f = exp2f(lds_m[ww][h] - M);
      L += lds_l[ww][h] * f;
      A += lds_acc[ww][h][d] * f;
    }
    if (a.S == 1) {
      const float o = L > 0.0f ? A / L : (a.empty_nan ? NAN : 0.0f);
      store_out<T>((T*)a.out + (row * a.Hq + (int64_t)g * GQ + h) * D + d, o);
    } else {
      part[2 * GQ + h * D + d] = A;
      if (d == 0) { part[h] = M; part[GQ + h] = L; }
    }
  }
  if (a.S == 1) return;

  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) is_last = (atomicAdd(&a.ws_count[i], 1) == a.S - 1);
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  if (threadIdx.x == 0) a.ws_count[i] = 0;
  const float* parts = a.ws_part + i * a.S * (int64_t)(GQ * (D + 2));
  const int stride = GQ * (D + 2);
  for (int j = threadIdx.x; j < GQ * D; j += LSA_BLOCK) {
    const int h = j / D, d = j % D;
    float M = kNegBig;
    for (int ss = 0; ss < a.S; ++ss) M = fmaxf(M, parts[ss * stride + h]);
    float L = 0.0f, A = 0.0f;
    for (int ss = 0; ss < a.S; ++ss) {
      const float* p = parts + ss * stride;
      const float f = exp2f(p[h] - M);
      L += p[GQ + h] * f;
      A += p[2 * GQ + h * D + d] * f;
    }
    const float o = L > 0.0f ? A / L : (a.empty_nan ? NAN : 0.0f);
    store_out<T>((T*)a.out + (row * a.Hq + (int64_t)g * GQ + h) * D + d, o);
  }
}

template <typename T, int D>
int launch_read_gq(const ReadArgs& a, int gq, dim3 grid, hipStream_t s) {
  switch (gq) {
    case 1: read_kernel<T, D, 1><<<grid, LSA_BLOCK, 0, s>>>(a); break;
    case 2: read_kernel<T, D, 2><<<grid, LSA_BLOCK, 0, s>>>(a); break;
    case 4: read_kernel<T, D, 4><<<grid, LSA_BLOCK, 0, s>>>(a); break;
    default: read_kernel<T, D, 8><<<grid, LSA_BLOCK, 0, s>>>(a); break;
  }
  return LSA_OK;
}

template <typename T>
int launch_read(const ReadArgs& a, int D, int gq, dim3 grid, hipStream_t s) {
  switch (D) {
    case 32: return launch_read_gq<T, 32>(a, gq, grid, s);
    case 64: return launch_read_gq<T, 64>(a, gq, grid, s);
    case 128: return launch_read_gq<T, 128>(a, gq, grid, s);
    default: return launch_read_gq<T, 256>(a, gq, grid, s);
  }
}

int check_read_common(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t Tq, int64_t Tk,
                      int32_t Hq, int32_t Hkv, int32_t D, const int32_t* ids, const int32_t* lengths, int32_t W,
                      const void* out) {
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
  return LSA_OK;
}

}  // namespace

extern "C" size_t lsa_read_scratch_bytes(int64_t rows, int32_t Hq, int32_t Hkv, int32_t D, int32_t splits) {
  if (splits <= 1 || rows <= 0 || Hkv <= 0 || Hq <= 0) return 0;
  const int64_t n = rows * Hkv;
  const int64_t gq = Hq / Hkv;
  return (size_t)n * splits * (size_t)(gq * (D + 2)) * sizeof(float);
}

extern "C" int lsa_read(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t Tq, int64_t Tk,
                        int32_t Hq, int32_t Hkv, int32_t D, const int32_t* ids, const int32_t* lengths, int32_t W,
                        int ids_per_head, float scale, int empty_nan, int32_t splits, int32_t* counters,
                        void* scratch, size_t scratch_bytes, void* out, void* stream) {
  int rc = check_read_common(q, k, v, dtype, B, Tq, Tk, Hq, Hkv, D, ids, lengths, W, out);
  if (rc != LSA_OK) return rc;
  LSA_REQUIRE(splits >= 1 && splits <= 1024, LSA_ERR_SHAPE, "lsa_read: splits in [1, 1024], got %d", splits);
  const int64_t rows = B * Tq;
  LSA_REQUIRE(rows * Hkv <= 0x7FFFFFFF, LSA_ERR_SHAPE, "lsa_read: too many rows");
  const size_t need = lsa_read_scratch_bytes(rows, Hq, Hkv, D, splits);
  LSA_REQUIRE(need == 0 || (scratch && counters && scratch_bytes >= need), LSA_ERR_WORKSPACE,
              "lsa_read: counters/scratch missing or scratch %zu < %zu bytes", scratch_bytes, need);
  if (rows * Hkv == 0) return LSA_OK;
  ReadArgs a;
  a.q = q; a.k = k; a.v = v; a.out = out; a.ids = ids; a.lengths = lengths;
  a.Tq = Tq; a.Tk = Tk; a.Hq = Hq; a.Hkv = Hkv; a.W = W; a.ids_per_head = ids_per_head ? 1 : 0; a.chunk = 0;
  a.scale_log2 = scale * kLog2e; a.empty_nan = empty_nan ? 1 : 0; a.S = splits;
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

// Chunked prefill through the gather kernel (one workgroup per (row, kv-head)); the
// MFMA tile kernel in read_prefill.hip serves bf16 at head dim 128.
static int lsa_read_chunked_gather(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t T, int64_t Tk,
                            int32_t Hq, int32_t Hkv, int32_t D, const int32_t* ids, const int32_t* lengths, int32_t W,
                            int32_t chunk, float scale, void* out, hipStream_t s) {
  ReadArgs a;
  a.q = q; a.k = k; a.v = v; a.out = out; a.ids = ids; a.lengths = lengths;
  a.Tq = T; a.Tk = Tk; a.Hq = Hq; a.Hkv = Hkv; a.W = W; a.ids_per_head = 1; a.chunk = chunk;
  a.scale_log2 = scale * kLog2e; a.empty_nan = 0; a.S = 1; a.ws_count = nullptr; a.ws_part = nullptr;
  const dim3 grid((unsigned)(B * T * Hkv), 1u);
  const int gq = Hq / Hkv;
  if (dtype == LSA_BF16) launch_read<bf16_t>(a, D, gq, grid, s);
  else if (dtype == LSA_F16) launch_read<_Float16>(a, D, gq, grid, s);
  else launch_read<float>(a, D, gq, grid, s);
  LSA_LAUNCHED("lsa_read_chunked");
  return LSA_OK;
}

extern "C" int lsa_read_chunked(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t T,
                                int64_t Tk, int32_t Hq, int32_t Hkv, int32_t D, const int32_t* ids,
                                const int32_t* lengths, int32_t W, int32_t chunk, float scale, void* out,
                                void* stream) {
  int rc = check_read_common(q, k, v, dtype, B, T, Tk, Hq, Hkv, D, ids, lengths, W, out);
  if (rc != LSA_OK) return rc;
  LSA_REQUIRE(chunk >= 1, LSA_ERR_SHAPE, "lsa_read_chunked: chunk must be >= 1");
  LSA_REQUIRE(T <= Tk, LSA_ERR_SHAPE, "lsa_read_chunked: %lld query rows exceed the cache %lld", (long long)T,
              (long long)Tk);
  LSA_REQUIRE(B * T * Hkv <= 0x7FFFFFFF, LSA_ERR_SHAPE, "lsa_read_chunked: too many rows");
  if (B * T * Hkv == 0) return LSA_OK;
  return lsa_read_chunked_gather(q, k, v, dtype, B, T, Tk, Hq, Hkv, D, ids, lengths, W, chunk, scale, out,
                                 (hipStream_t)stream);
}
