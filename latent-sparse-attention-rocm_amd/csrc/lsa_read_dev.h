// Device code of the sparse gather read, shared by the read kernel and the fused decode
// kernel: row loads and conversions, lane reductions, the tile loop of one list span
// (online softmax over gathered K/V rows), the wave merge, and the split-K partial
// publish / combine.
#pragma once

#include <math.h>

#include "lsa_device.h"

namespace lsa {

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

// exp2 on the hardware unit (v_exp_f32): softmax weights that would be denormal flush
// to zero, which the normaliser never notices.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

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
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
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


// LDS of the read finish: per-wave states, split weights, reduction buffers.
template <int D, int GQ, int MAXS>
struct ReadLds {
  static constexpr int COLS = GQ * D / 4;
  static constexpr int RPT = COLS >= LSA_BLOCK ? 1 : LSA_BLOCK / COLS;
  float acc[LSA_WAVES][GQ][D];
  float m[LSA_WAVES][GQ];
  float l[LSA_WAVES][GQ];
  float w[MAXS][GQ];
  float pl[MAXS][GQ];
  float ltot[GQ];
  float4 red[RPT > 1 ? RPT : 1][RPT > 1 ? COLS : 1];
  int flag;
};

// Which instances score on the matrix cores: 16-bit rows of D = 128 (tiles of 64 slots,
// 16 lanes a row) for up to 8 query heads a kv-head.
template <typename T, int D, int GQ>
struct ReadMfma {
  static constexpr bool ON = sizeof(T) == 2 && D == 128 && GQ <= 8 && ReadShape<T, D, GQ>::NT == 64 &&
                             ReadShape<T, D, GQ>::LPT == 16;
};

// 16x16x32 MFMA on 8 packed 16-bit elements a lane, fp32 accumulate.
template <typename T> struct Mfma16;
template <> struct Mfma16<bf16_t> {
  static __device__ __forceinline__ f32x4_t run(const uint4& a, const uint4& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  }
};
template <> struct Mfma16<_Float16> {
  static __device__ __forceinline__ f32x4_t run(const uint4& a, const uint4& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  }
};

// The GQ query rows of one kv-head as this lane holds them: raw 16-byte words (16-bit
// rows score with packed dot products on them, the scale applied to the fp32 sum) and, for
// fp32 rows, floats pre-scaled by scale_log2. qrow points at the GQ contiguous rows. For
// the matrix-core score, qm is the B operand of S^T = K Q^T: lane (row = lane / 16,
// col = lane % 16) holds dims 32 i + 8 row .. + 8 of query head col (zeros for col >= GQ)
// for the i-th 32-dim quarter.
template <typename T, int D, int GQ>
struct QueryRegs {
  static constexpr bool PACKED = sizeof(T) == 2;
  uint32_t qw[GQ][4];
  float qf[GQ][ReadShape<T, D, GQ>::VEC];
  uint4 qm[D / 32 > 0 ? D / 32 : 1];

  __device__ __forceinline__ void load(const T* qrow, float scale_log2) {
    using S = ReadShape<T, D, GQ>;
    if constexpr (ReadMfma<T, D, GQ>::ON) {
      const int lane = threadIdx.x & (LSA_WAVE - 1), row = lane >> 4, col = lane & 15;
      const T* src = qrow + (int64_t)(col < GQ ? col : 0) * D + 8 * row;
#pragma unroll
      for (int i = 0; i < D / 32; ++i) {
        const uint4 x = *(const uint4*)(src + 32 * i);
        qm[i] = col < GQ ? x : make_uint4(0u, 0u, 0u, 0u);
      }
      return;
    }
    const int lp = (threadIdx.x & (LSA_WAVE - 1)) % S::LPT;
#pragma unroll
    for (int h = 0; h < GQ; ++h) {
      const uint4 raw = *(const uint4*)(qrow + (int64_t)h * D + lp * S::VEC);
      qw[h][0] = raw.x; qw[h][1] = raw.y; qw[h][2] = raw.z; qw[h][3] = raw.w;
      if constexpr (!PACKED) {
        Row16<T>::cvt(raw, qf[h]);
#pragma unroll
        for (int e = 0; e < S::VEC; ++e) qf[h][e] *= scale_log2;
      }
    }
  }
};

// Per-lane running softmax state of the GQ heads over this lane's VEC dims.
template <typename T, int D, int GQ>
struct AttnState {
  float m[GQ], l[GQ], acc[GQ][ReadShape<T, D, GQ>::VEC];

  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int h = 0; h < GQ; ++h) {
      m[h] = kNegBig;
      l[h] = 0.0f;
#pragma unroll
      for (int e = 0; e < ReadShape<T, D, GQ>::VEC; ++e) acc[h][e] = 0.0f;
    }
  }
};

// attend_tiles for the matrix-core instances (ReadMfma::ON). Wave w takes slots
// [16 w, 16 w + 16) of each 64-slot tile. S^T (16 tokens x 16 query columns, GQ real) =
// K Q^T is four 16x16x32 MFMAs, one a 32-dim quarter: lane (row, col) loads dims
// 32 i + 8 row .. + 8 of token col's K row. In the accumulator, lane (row, col) holds
// tokens 4 row + u (u < 4) of head col, so a head's tile maximum is a max over four
// registers and two lane swaps. The running maximum moves only when a tile's exceeds it
// by more than 2^8 (weights stay below 256, exact in fp32), and only then is the state
// rescaled. Weights reach the V side through a 16 x GQ LDS block per wave: lane (row, lp)
// holds V dims 8 lp .. + 8 of tokens 4 row + u, the tokens of its own accumulator row,
// so a masked token's weight is already 0 there. The state leaves in the layout of the
// other instances (m uniform, l and acc per token group).
//
// With PIPE, spans of two tiles or more are software-pipelined: tile t + 1's K/V loads are issued
// before tile t is computed, and each lane's slot id is fetched two tiles ahead, ahead of
// the loads it does not feed (memory counters retire in order, so a wait for an id must
// not also wait for the rows in flight). The V side's ids come from the K side's by lane
// permutes. Slots past the span read -1 (a partial last tile): those rows load token 0
// (cache hits) and weigh nothing.
template <typename T, int D, int GQ>
struct MfmaTile {
  static constexpr int NM = D / 32;
  uint4 k[NM], v[4];
  bool ok[4];
};

template <typename T, int D, int GQ, bool PIPE, typename IdOf>
__device__ __forceinline__ void attend_tiles_mfma(const QueryRegs<T, D, GQ>& q, const T* kb, const T* vb,
                                                  int64_t tstride, int64_t Tk, int lo, int hi, IdOf id_of,
                                                  float scale_log2, AttnState<T, D, GQ>& st) {
  constexpr int NM = D / 32, NT = ReadShape<T, D, GQ>::NT, VEC = ReadShape<T, D, GQ>::VEC;
  constexpr float kLazy = 8.0f;  // log2 growth of a head's maximum that forces a rescale
  __shared__ __attribute__((aligned(16))) float pw[LSA_WAVES][16][GQ];
  const int lane = threadIdx.x & (LSA_WAVE - 1), w = threadIdx.x / LSA_WAVE;
  const int row = lane >> 4, col = lane & 15;
  const T* kq = kb + 8 * (row - col);  // kb points at this lane's V dims (8 col)
  const int s0 = 16 * w + col;         // this lane's slot (K side) within a tile
  float mrun = st.m[0], lrun = st.l[0];  // head col's running max; its sum over this row's tokens
#pragma unroll
  for (int h = 1; h < GQ; ++h) {
    mrun = col == h ? st.m[h] : mrun;
    lrun = col == h ? st.l[h] : lrun;
  }

  auto issue = [&](int32_t idk, MfmaTile<T, D, GQ>& t) {
    const bool okk = idk >= 0 && idk < Tk;
    const uint64_t koff = (uint64_t)(uint32_t)(okk ? idk : 0) * (uint32_t)tstride;
#pragma unroll
    for (int i = 0; i < NM; ++i) t.k[i] = *(const uint4*)(kq + koff + 32 * i);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int32_t idv = __shfl(idk, 4 * row + u, LSA_WAVE);  // token 4 row + u's id
      const bool okv = idv >= 0 && idv < Tk;
      t.ok[u] = okv && col < GQ;
      t.v[u] = *(const uint4*)(vb + (uint64_t)(uint32_t)(okv ? idv : 0) * (uint32_t)tstride);
    }
  };
  auto compute = [&](const MfmaTile<T, D, GQ>& t) {
    f32x4_t c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NM; ++i) c = Mfma16<T>::run(t.k[i], q.qm[i], c);
    float s[4], mt = -INFINITY;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      s[u] = t.ok[u] ? c[u] * scale_log2 : -INFINITY;
      mt = fmaxf(mt, s[u]);
    }
    mt = fmaxf(mt, lane_xor(mt, 16));
    mt = fmaxf(mt, lane_xor(mt, 32));
    if (__ballot(mt > mrun + kLazy) != 0) {  // wave-uniform: some head's maximum moved
      const float mnew = fmaxf(mrun, mt);
      const float alpha = fast_exp2(mrun - mnew);
      mrun = mnew;
      lrun *= alpha;
#pragma unroll
      for (int h = 0; h < GQ; ++h) {
        const float ah = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), h));
#pragma unroll
        for (int e = 0; e < VEC; ++e) st.acc[h][e] *= ah;
      }
    }
    float p[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      p[u] = fast_exp2(s[u] - mrun);  // 0 for masked tokens and padded heads
      lrun += p[u];
    }
    if (col < GQ) {
#pragma unroll
      for (int u = 0; u < 4; ++u) pw[w][4 * row + u][col] = p[u];
    }
    __builtin_amdgcn_wave_barrier();  // the wave's LDS writes before its reads
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float ph[GQ];
#pragma unroll
      for (int h = 0; h < GQ; ++h) ph[h] = pw[w][4 * row + u][h];
      float vf[VEC];
      Row16<T>::cvt(t.v[u], vf);
#pragma unroll
      for (int h = 0; h < GQ; ++h) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) st.acc[h][e] = fmaf(ph[h], vf[e], st.acc[h][e]);
      }
    }
    __builtin_amdgcn_wave_barrier();  // the reads before the next tile's writes
  };

  // the span is wave-uniform: scalar bounds make the tile loop's tests scalar branches
  lo = __builtin_amdgcn_readfirstlane(lo);
  hi = __builtin_amdgcn_readfirstlane(hi);
  if (PIPE && hi - lo > NT) {  // pipelined
    // Two tile buffers that trade roles every tile (the loop body holds two tiles): the
    // next tile's rows land in the other buffer while this one is computed. A copy from
    // a "next" buffer into a "current" one would wait for the rows in flight, which
    // leaves one tile's gather exposed every iteration.
    MfmaTile<T, D, GQ> ta, tb;
    // One exit, at the loop's head: a loop with exits in its middle is folded into one exit
    // behind a flow block that re-enters the head with rows still in flight, and the head
    // then waits for all of them.
    const int n_tiles = (hi - lo + NT - 1) / NT;  // >= 2
    int32_t id_a = id_of(lo + s0);
    int32_t id_b = id_of(lo + NT + s0);
    issue(id_a, ta);
    int base = lo;
    for (int t = 0; t + 2 < n_tiles; t += 2, base += 2 * NT) {  // ta holds tile t; t + 1, t + 2 exist
      id_a = id_of(base + 2 * NT + s0);  // ids two tiles ahead, before the rows they do not feed
      issue(id_b, tb);
      compute(ta);
      id_b = id_of(base + 3 * NT + s0);
      issue(id_a, ta);
      compute(tb);
    }
    if (base + NT < hi) {  // uniform: one more tile after ta's
      issue(id_b, tb);
      compute(ta);
      compute(tb);
    } else {
      compute(ta);
    }
  } else {
    MfmaTile<T, D, GQ> cur;
    int32_t id1 = id_of(lo + s0);
    for (int base = lo; base < hi; base += NT) {
      issue(id1, cur);
      id1 = id_of(base + NT + s0);  // next tile's id while this one computes
      compute(cur);
    }
  }
#pragma unroll
  for (int h = 0; h < GQ; ++h) {
    st.m[h] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mrun), h));
    st.l[h] = __shfl(lrun, 16 * row + h, LSA_WAVE);
  }
}

// Online-softmax attention over list slots [lo, hi), tile by tile: id_of(j) is the token of
// slot j, or -1 (skipped); it must be cheap and unconditional (a clamped load or an LDS
// read). kb / vb point at the kv-head's row 0 plus this lane's VEC-element offset. fresh:
// the state is empty, so the first tile needs no rescale.
template <typename T, int D, int GQ, bool PIPE = false, typename IdOf>
__device__ __forceinline__ void attend_tiles(const QueryRegs<T, D, GQ>& q, const T* kb, const T* vb, int64_t tstride,
                                             int64_t Tk, int lo, int hi, IdOf id_of, float scale_log2, bool fresh,
                                             AttnState<T, D, GQ>& st) {
  if constexpr (ReadMfma<T, D, GQ>::ON) {
    attend_tiles_mfma<T, D, GQ, PIPE>(q, kb, vb, tstride, Tk, lo, hi, id_of, scale_log2, st);
    return;
  }
  using S = ReadShape<T, D, GQ>;
  constexpr int VEC = S::VEC, LPT = S::LPT, TPW = S::TPW, U = S::U, NT = S::NT;
  constexpr bool PACKED = QueryRegs<T, D, GQ>::PACKED;
  const int lane = threadIdx.x & (LSA_WAVE - 1);
  const int w = threadIdx.x / LSA_WAVE;
  const int tg = lane / LPT;

  int32_t id[U];
#pragma unroll
  for (int u = 0; u < U; ++u) id[u] = id_of(lo + (u * LSA_WAVES + w) * TPW + tg);
  for (int base = lo; base < hi; base += NT) {
    // all K/V rows of the tile in flight at once
    bool ok[U];
    uint4 kr[U], vr[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ok[u] = id[u] >= 0 && id[u] < Tk;
      const uint64_t off = (uint64_t)(uint32_t)(ok[u] ? id[u] : 0) * (uint32_t)tstride;
      kr[u] = *(const uint4*)(kb + off);
      vr[u] = *(const uint4*)(vb + off);
    }
    // next tile's ids while this one computes
    const int nb = base + NT;
#pragma unroll
    for (int u = 0; u < U; ++u) id[u] = id_of(nb + (u * LSA_WAVES + w) * TPW + tg);

    float sc[GQ][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int h = 0; h < GQ; ++h) {
        float p;
        if constexpr (PACKED) {
          p = dot8<T>(q.qw[h], kr[u]);
        } else {
          float kf[VEC];
          Row16<T>::cvt(kr[u], kf);
          p = 0.0f;
#pragma unroll
          for (int e = 0; e < VEC; ++e) p = fmaf(q.qf[h][e], kf[e], p);
        }
        p = group_sum<LPT>(p);
        if constexpr (PACKED) p *= scale_log2;
        sc[h][u] = ok[u] ? p : -INFINITY;
      }
    }
    const bool rescale = !(fresh && base == lo);  // an empty state needs no rescale
#pragma unroll
    for (int h = 0; h < GQ; ++h) {
      float mt = st.m[h];
#pragma unroll
      for (int u = 0; u < U; ++u) mt = fmaxf(mt, sc[h][u]);
      if (rescale) {
        const float alpha = fast_exp2(st.m[h] - mt);
        st.l[h] *= alpha;
#pragma unroll
        for (int e = 0; e < VEC; ++e) st.acc[h][e] *= alpha;
      }
      st.m[h] = mt;
#pragma unroll
      for (int u = 0; u < U; ++u) sc[h][u] = fast_exp2(sc[h][u] - mt);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float vf[VEC];
      Row16<T>::cvt(vr[u], vf);
#pragma unroll
      for (int h = 0; h < GQ; ++h) {
        st.l[h] += sc[h][u];
#pragma unroll
        for (int e = 0; e < VEC; ++e) st.acc[h][e] = fmaf(sc[h][u], vf[e], st.acc[h][e]);
      }
    }
  }
}

// Merges the token groups of each wave (lanes that hold the same dims): afterwards every
// lane of a group holds the wave's state for its dims.
template <typename T, int D, int GQ>
__device__ __forceinline__ void merge_token_groups(AttnState<T, D, GQ>& st) {
  using S = ReadShape<T, D, GQ>;
  constexpr int VEC = S::VEC, LPT = S::LPT;
#pragma unroll
  for (int x = LPT; x < LSA_WAVE; x <<= 1) {
#pragma unroll
    for (int h = 0; h < GQ; ++h) {
      const float mo = lane_xor(st.m[h], x);
      const float lo_ = lane_xor(st.l[h], x);
      const float mn = fmaxf(st.m[h], mo);
      const float a1 = fast_exp2(st.m[h] - mn), a2 = fast_exp2(mo - mn);
      st.l[h] = st.l[h] * a1 + lo_ * a2;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float ao = lane_xor(st.acc[h][e], x);
        st.acc[h][e] = st.acc[h][e] * a1 + ao * a2;
      }
      st.m[h] = mn;
    }
  }
}

// Attention of the GQ query heads of one kv-head over list slots [lo, hi) from an empty
// state, token groups merged (qrow: the GQ contiguous query rows).
template <typename T, int D, int GQ, typename IdOf>
__device__ __forceinline__ void attend_span(const T* qrow, const T* kb, const T* vb, int64_t tstride, int64_t Tk,
                                            int lo, int hi, IdOf id_of, float scale_log2, AttnState<T, D, GQ>& st) {
  QueryRegs<T, D, GQ> q;
  q.load(qrow, scale_log2);
  st.clear();
  attend_tiles<T, D, GQ, true>(q, kb, vb, tstride, Tk, lo, hi, id_of, scale_log2, true, st);
  merge_token_groups<T, D, GQ>(st);
}

// Sums each of N values (N % 4 == 0) over the four 16-lane rows of the wave by two rounds
// of row swaps, each swap serving two values: after the 16-row swap of values a and b, one
// register holds rows [a0, b0, a2, b2] and the other [a1, b1, a3, b3], whose sum packs two
// half-reductions into one register; the 32-row swap of two such registers does the same
// for the row pairs. Value v's wave total lands in out[v / 4], row v % 4 (every lane of
// that row, for its own column): 1.5 N instructions instead of the 4 N of a butterfly that
// keeps every value in every row.
template <int N>
__device__ __forceinline__ void row_transpose_sum(const float (&x)[N], float (&out)[N / 4]) {
  static_assert(N % 4 == 0, "row_transpose_sum packs four values a register");
  float half[N / 2];
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    float a = x[2 * i], b = x[2 * i + 1];
    row_swap16(a, b);
    half[i] = a + b;
  }
#pragma unroll
  for (int i = 0; i < N / 4; ++i) {
    float a = half[2 * i], b = half[2 * i + 1];
    row_swap32(a, b);
    out[i] = a + b;
  }
}

// Merges the token groups of each wave and then the four waves' states of a span (st: a
// lane's state as attend_tiles leaves it). direct: writes the normalised output to outp
// (GQ rows of D); otherwise publishes the partial (m[GQ], l[GQ], acc[GQ][D]) at part with
// write-through stores. Every thread calls it.
template <typename T, int D, int GQ, int MAXS, bool MERGED = false>
__device__ __forceinline__ void finish_span(ReadLds<D, GQ, MAXS>& sh, AttnState<T, D, GQ>& st, bool direct,
                                            T* outp, float* part, int empty_nan) {
  using S = ReadShape<T, D, GQ>;
  constexpr int VEC = S::VEC, LPT = S::LPT;
  const int lane = threadIdx.x & (LSA_WAVE - 1);
  const int w = threadIdx.x / LSA_WAVE;
  const int tg = lane / LPT, lp = lane % LPT;
  constexpr bool ON = ReadMfma<T, D, GQ>::ON && !MERGED;
  // matrix-core instances: the accumulators in LDS as the row-transposed sums leave them,
  // register i of lane l of wave w at stage[(w * NA + i) * 64 + l] (within sh.acc)
  constexpr int NA = GQ * VEC / 4;
  float* stage = &sh.acc[0][0][0];
  if constexpr (ON) {
    // one running maximum per head for the whole wave (the token groups are the four
    // 16-lane rows): the groups merge by sums, packed four values a register, stored as
    // whole wave rows (conflict-free)
    float x[GQ * VEC], tot[NA];
#pragma unroll
    for (int h = 0; h < GQ; ++h) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) x[h * VEC + e] = st.acc[h][e];
    }
    row_transpose_sum<GQ * VEC>(x, tot);
#pragma unroll
    for (int i = 0; i < NA; ++i) stage[(w * NA + i) * LSA_WAVE + lane] = tot[i];
    constexpr int NL = (GQ + 3) / 4 * 4;
    float xl[NL], tl[NL / 4];
#pragma unroll
    for (int h = 0; h < NL; ++h) xl[h] = h < GQ ? st.l[h] : 0.0f;
    row_transpose_sum<NL>(xl, tl);
#pragma unroll
    for (int i = 0; i < NL / 4; ++i) {
      if (lp == 0 && 4 * i + tg < GQ) sh.l[w][4 * i + tg] = tl[i];
    }
    if (lane == 0) {  // the maxima are uniform over the wave (static indices keep st in registers)
#pragma unroll
      for (int h = 0; h < GQ; ++h) sh.m[w][h] = st.m[h];
    }
  } else {
    if constexpr (!MERGED) merge_token_groups<T, D, GQ>(st);
    if (tg == 0) {
#pragma unroll
      for (int h = 0; h < GQ; ++h) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) sh.acc[w][h][lp * VEC + e] = st.acc[h][e];
        if (lp == 0) { sh.m[w][h] = st.m[h]; sh.l[w][h] = st.l[h]; }
      }
    }
  }
  __syncthreads();
  // thread j owns (head, dim) pairs j, j + 256, ...
  for (int j = threadIdx.x; j < GQ * D; j += LSA_BLOCK) {
    const int h = j / D, d = j % D;
    float M = kNegBig;
#pragma unroll
    for (int ww = 0; ww < LSA_WAVES; ++ww) M = fmaxf(M, sh.m[ww][h]);
    float L = 0.0f, A = 0.0f;
    // the staged slot of (h, d): value v = h VEC + d % VEC of column d / VEC, register v / 4
    // of row v % 4
    const int v = h * VEC + d % VEC;
    const int slot = (v / 4) * LSA_WAVE + 16 * (v % 4) + d / VEC;
#pragma unroll
    for (int ww = 0; ww < LSA_WAVES; ++ww) {
      const float f = fast_exp2(sh.m[ww][h] - M);
      L += sh.l[ww][h] * f;
      A += (ON ? stage[ww * NA * LSA_WAVE + slot] : sh.acc[ww][h][d]) * f;
    }
    if (direct) {
      store_out<T>(outp + j, L > 0.0f ? A / L : (empty_nan ? NAN : 0.0f));
    } else {
      coherent_store(part + 2 * GQ + j, A);
      if (d == 0) { coherent_store(part + h, M); coherent_store(part + GQ + h, L); }
    }
  }
}

// Combines n_act published partials (stride GQ*(D+2) floats from parts) into outp. The
// first batch of accumulator columns and every (m, l) are loaded together; per-head
// maxima and normalisers are wave reductions (a fixed order: deterministic). Every
// thread calls it; n_act <= MAXS.
template <typename T, int D, int GQ, int MAXS>
__device__ __forceinline__ void combine_partials(ReadLds<D, GQ, MAXS>& sh, const float* parts, int n_act, T* outp,
                                                 int empty_nan) {
  constexpr int COLS = GQ * D / 4;                                // float4 columns of a partial
  constexpr int RPT = COLS >= LSA_BLOCK ? 1 : LSA_BLOCK / COLS;   // threads per column
  constexpr int CPT = COLS >= LSA_BLOCK ? COLS / LSA_BLOCK : 1;   // columns per thread
  constexpr int PSTRIDE = GQ * (D + 2);
  constexpr int BATCH = 16 / CPT;
  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1), w = tid / LSA_WAVE;
  const int r = tid / COLS % RPT;
  const CoherentRows rows(parts);  // partials of one unit span < 2 GiB
  float4 first[CPT][BATCH];
#pragma unroll
  for (int cc = 0; cc < CPT; ++cc) {
    const int c = (tid % COLS) + cc * LSA_BLOCK;
#pragma unroll
    for (int bb = 0; bb < BATCH; ++bb) {
      const int sp = r + bb * RPT;
      const int sl = sp < n_act ? sp : 0;
      first[cc][bb] = rows.load4(4 * (sl * PSTRIDE + 2 * GQ + 4 * c));
    }
  }
  for (int t = tid; t < n_act * GQ; t += LSA_BLOCK) {
    const int sp = t / GQ, h = t % GQ;
    const float* ps = parts + (int64_t)sp * PSTRIDE;
    const float pm = coherent_load(ps + h), pl = coherent_load(ps + GQ + h);
    sh.w[sp][h] = pm;
    sh.pl[sp][h] = pl;
  }
  __syncthreads();
  // per-head maximum and normaliser: wave w reduces heads w, w + 4, ... with the splits
  // strided over its lanes
  for (int h = w; h < GQ; h += LSA_WAVES) {
    float M = kNegBig;
    for (int sp = lane; sp < n_act; sp += LSA_WAVE) M = fmaxf(M, sh.w[sp][h]);
    M = wave_max(M);
    float L = 0.0f;
    for (int sp = lane; sp < n_act; sp += LSA_WAVE) {
      const float f = fast_exp2(sh.w[sp][h] - M);
      L += sh.pl[sp][h] * f;
      sh.w[sp][h] = f;
    }
    L = wave_sum(L);
    if (lane == 0) sh.ltot[h] = L;
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
      const float f = sp < n_act ? sh.w[sp][h] : 0.0f;
      sum.x += f * first[cc][bb].x; sum.y += f * first[cc][bb].y;
      sum.z += f * first[cc][bb].z; sum.w += f * first[cc][bb].w;
    }
    for (int sb = BATCH * RPT; sb < n_act; sb += BATCH * RPT) {  // more splits than one batch
      float4 x[BATCH];
#pragma unroll
      for (int bb = 0; bb < BATCH; ++bb) {
        const int sp = r + sb + bb * RPT;
        x[bb] = rows.load4(4 * ((sp < n_act ? sp : 0) * PSTRIDE + 2 * GQ + 4 * c));
      }
#pragma unroll
      for (int bb = 0; bb < BATCH; ++bb) {
        const int sp = r + sb + bb * RPT;
        const float f = sp < n_act ? sh.w[sp][h] : 0.0f;
        sum.x += f * x[bb].x; sum.y += f * x[bb].y; sum.z += f * x[bb].z; sum.w += f * x[bb].w;
      }
    }
    if (RPT > 1) {
      sh.red[r][c] = sum;
    } else {
      const float L = sh.ltot[h];
      const float inv = L > 0.0f ? 1.0f / L : 0.0f;
      const float e = empty_nan ? NAN : 0.0f;
      store_out<T>(outp + 4 * c + 0, L > 0.0f ? sum.x * inv : e);
      store_out<T>(outp + 4 * c + 1, L > 0.0f ? sum.y * inv : e);
      store_out<T>(outp + 4 * c + 2, L > 0.0f ? sum.z * inv : e);
      store_out<T>(outp + 4 * c + 3, L > 0.0f ? sum.w * inv : e);
    }
  }
  if (RPT > 1) {
    __syncthreads();
    for (int c = tid; c < COLS; c += LSA_BLOCK) {
      float4 sum = sh.red[0][c];
#pragma unroll
      for (int rr = 1; rr < RPT; ++rr) {
        const float4 x = sh.red[rr][c];
        sum.x += x.x; sum.y += x.y; sum.z += x.z; sum.w += x.w;
      }
      const int h = (4 * c) / D;
      const float L = sh.ltot[h];
      const float inv = L > 0.0f ? 1.0f / L : 0.0f;
      const float e = empty_nan ? NAN : 0.0f;
      store_out<T>(outp + 4 * c + 0, L > 0.0f ? sum.x * inv : e);
      store_out<T>(outp + 4 * c + 1, L > 0.0f ? sum.y * inv : e);
      store_out<T>(outp + 4 * c + 2, L > 0.0f ? sum.z * inv : e);
      store_out<T>(outp + 4 * c + 3, L > 0.0f ? sum.w * inv : e);
    }
  }
}

}  // namespace lsa
