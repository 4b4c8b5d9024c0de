// MFMA tile kernel for the chunked prefill read (16-bit rows, head dim 64 or 128).
//
// Query row t of chunk c = t / chunk reads chunk c's per-kv-head list (its first lengths
// slots) and then the chunk's own causal block [c*chunk, t] (the reference read of the
// chunked prefill: read_kernel_tiled.py:30-89 over these lists). Every row of a chunk
// shares the list, so one workgroup serves (batch, chunk, kv-head, head group): the
// chunk's rows of up to 256 / chunk query heads of the group - 256 query rows, 32 per
// wave - and every K/V row of the list is gathered once for all of them.
//
// Per 64-key tile: the K and V rows land in LDS row-major (four tile buffers: two being
// read, one being stored, one free), gathered a tile ahead of their store, from inside the
// math of the tile before. Each wave computes S^T = K Q^T a 32-key sub-tile at a time
// (v_mfma_f32_32x32x16: the K rows are the A operand read straight from LDS, Q^T the B
// operand held in registers for the whole kernel), masks skipped and non-causal keys where
// the sub-tile has any, runs the online softmax in the exp2 domain per query column, and
// accumulates O^T += V^T P^T: the S^T accumulator layout is exactly the P^T B operand
// (lane (h, q) holds keys 8(r/4) + 4h + r%4 of column q), so P needs no shuffle; the V^T
// A operand comes from the row-major V tile through transposing LDS reads. A wave's
// sub-tiles are software-pipelined three deep: while the matrix core forms the next
// sub-tile's scores and the previous sub-tile's P V product, the VALU makes this
// sub-tile's weights. The running max is rescaled lazily: only when a column's max grows by
// more than 2^8 is the state rescaled, so P stays below 256 in the 16-bit operand and most
// tiles skip the 128-register rescale; the weights are made against the current max
// first, and the column maxima are taken only when some lane's weight sum reaches 2^8
// (which every such growth implies). The softmax normaliser sums the 16-bit weights the
// matrix ops use.
#include <math.h>

#include <type_traits>

#include "lsa_abi_common.h"
#include "lsa_read_dev.h"

using namespace lsa;

namespace {

constexpr int TK = 64;     // keys per staged tile (one barrier)
constexpr int TS = 32;     // keys per sub-tile (one 32 x 32 S^T block)
constexpr int KPAD = 8;    // LDS row padding of the K tile (elements)
constexpr int VPAD = 32;   // of the V tile: rows 16 dwords apart mod 64 banks (conflict-free transposed reads)
constexpr float kRescale = 8.0f;  // log2 growth of a column max that forces a rescale
constexpr int kRows = 256;       // query rows of a workgroup
constexpr int NBUF = 4;          // LDS tile buffers (two read, one being stored, one free)

typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <typename T> struct Mfma;
template <> struct Mfma<bf16_t> {
  typedef bf16x8_t op_t;
  static __device__ __forceinline__ f32x16_t run(op_t a, op_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {  // v_cvt_pk_bf16_f32 (RNE)
    typedef __bf16 v2_t __attribute__((ext_vector_type(2)));
    typedef float f2_t __attribute__((ext_vector_type(2)));
    const f2_t f = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, v2_t));
  }
  // c + lo + hi of a packed pair (v_dot2_f32_bf16 against ones)
  static __device__ __forceinline__ float sum2(uint32_t pair, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pair), __builtin_bit_cast(bf16x2_t, 0x3F803F80u),
                                           c, false);
  }
};
template <> struct Mfma<_Float16> {
  typedef f16x8_t op_t;
  static __device__ __forceinline__ f32x16_t run(op_t a, op_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    typedef _Float16 v2_t __attribute__((ext_vector_type(2)));
    typedef float f2_t __attribute__((ext_vector_type(2)));
    const f2_t f = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, v2_t));
  }
  static __device__ __forceinline__ float sum2(uint32_t pair, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, pair), __builtin_bit_cast(f16x2_t, 0x3C003C00u), c, false);
  }
};

template <int D>
struct alignas(16) PrefillLds {
  uint16_t k[NBUF][TK][D + KPAD];   // K rows, raw 16-bit elements
  uint16_t v[NBUF][TK][D + VPAD];   // V rows, raw 16-bit elements
  int info[NBUF][TK];               // per key: -2 skipped, -1 list key (every row), o >= 0 local offset
  int odd[NBUF][TK / TS];           // tile number whose sub-tile holds a key that is not a list key
};

// Four keys of one V column from the row-major V tile, for a V^T MFMA operand, by the
// transposing LDS read (ds_read_b64_tr_b16): in each group of 16 lanes, lane j addresses
// the 8 bytes at key0 + j / 4, dims dim0 + 4 (j % 4) .. + 3, and lane i receives keys
// key0 .. key0 + 3 of dim dim0 + i.
// `lane_base` is this lane's part of the address (key j / 4, dims 4 (j % 4) of the tile);
// the rest is a constant byte offset, which the read's immediate field takes.
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char lds_char;
__device__ __forceinline__ uint2 v_column4(const lds_char* lane_base, int offset) {
  typedef __attribute__((address_space(3))) v4i16_t lds_v4;
  const v4i16_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4*)(lane_base + offset));
  return __builtin_bit_cast(uint2, r);
}

struct PrefillArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  const int32_t* ids;
  const int32_t* lengths;
  int64_t T, Tk;
  int64_t kv_sb, kv_st, kv_sh;
  int Hq, Hkv, W, chunk, C;
  int hpw;   // query heads per workgroup (256 / chunk, at most the group)
  int n_hg;  // head groups per kv-head
  SlotMap slots;  // a paged cache: the causal block's positions -> cache rows
  float scale_log2;
};

// QB query blocks of 32 columns per wave; 8 / QB waves hold the workgroup's 256 rows.
template <typename T, int D, int QB, bool OFF32>
__global__ __launch_bounds__(64 * (8 / QB)) void prefill_mfma_kernel(PrefillArgs a) {
  using M = Mfma<T>;
  using op_t = typename M::op_t;
  constexpr int NTH = 64 * (8 / QB);      // threads
  constexpr int KS = D / 16;              // k-steps of S^T
  constexpr int DB = D / 32;              // dim blocks of O^T
  constexpr int SEGS = D / 8;             // 16-byte segments of a row
  constexpr int KPP = NTH / SEGS;         // keys loaded per pass
  constexpr int PASSES = TK >= KPP ? TK / KPP : 1;
  __shared__ PrefillLds<D> sh;

  const int tid = threadIdx.x, lane = tid & (LSA_WAVE - 1), w = tid / LSA_WAVE;
  const int hh = lane / 32, ln = lane % 32;
  // this lane's byte offset in a V tile for the transposing reads: keys 4 hh + (lane % 16) / 4,
  // dims 16 (ln / 16) + 4 (lane % 4)
  const int vlane = 2 * ((4 * hh + (lane % 16) / 4) * (D + VPAD) + 16 * (ln / 16) + 4 * (lane % 4));
  int64_t x = blockIdx.x;
  const int hg = (int)(x % a.n_hg); x /= a.n_hg;
  const int g = (int)(x % a.Hkv); x /= a.Hkv;
  const int c = a.C - 1 - (int)(x % a.C);  // later chunks see more buckets: longest first
  const int64_t b = x / a.C;
  const int gq = a.Hq / a.Hkv;
  const int64_t c0 = (int64_t)c * a.chunk;
  const int n_loc = (int)min((int64_t)a.chunk, a.T - c0);  // rows of this chunk
  const int64_t li = (b * a.C + c) * a.Hkv + g;
  int n_list = a.W > 0 ? a.lengths[li] : 0;
  n_list = n_list < 0 ? 0 : (n_list > a.W ? a.W : n_list);
  const int32_t* list = a.ids + li * a.W;
  const int n_tot = n_list + n_loc;
  const int n_tiles = (n_tot + TK - 1) / TK;
  const T* kb = (const T*)a.k + b * a.kv_sb + (int64_t)g * a.kv_sh;
  const T* vb = (const T*)a.v + b * a.kv_sb + (int64_t)g * a.kv_sh;
  // a paged cache (uniform): the causal block's positions go through the slot table row of
  // batch row b, fetched where the list ids are (the chunk lists already hold cache rows)
  const SlotRow smap = slot_row_of(a.slots, b);
  const bool paged = smap.row != nullptr;

  // this lane's query columns: qi = 32 QB w + 32 qb + ln -> (local head, token)
  int tok[QB];
  bool qok[QB];
  int64_t qrow[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int qi = 32 * QB * w + 32 * qb + ln;
    const int hl = qi / a.chunk;
    tok[qb] = qi % a.chunk;
    const int head_in_group = hg * a.hpw + hl;
    qok[qb] = hl < a.hpw && head_in_group < gq && tok[qb] < n_loc;
    const int head = g * gq + (qok[qb] ? head_in_group : 0);
    const int64_t t = c0 + (qok[qb] ? tok[qb] : 0);
    qrow[qb] = ((b * a.T + t) * a.Hq + head) * (int64_t)D;
  }
  // Q^T B operands, whole kernel: 16 bytes of row q at dims [16 s + 8 hh, +8)
  op_t qop[QB][KS];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint4 raw = *(const uint4*)((const T*)a.q + qrow[qb] + 16 * s + 8 * hh);
      qop[qb][s] = __builtin_bit_cast(op_t, raw);
    }
  }

  // tile loads: key kk = pass * KPP + tid / SEGS, segment seg = tid % SEGS. A tile's rows are
  // gathered one iteration before their store into LDS and its list ids one iteration
  // before that; both are issued from inside the math (between matrix ops) rather than as a
  // phase of their own, so the gathers and LDS writes overlap the matrix and vector work.
  // Loads past the last tile are clamped (unconditional loads keep every wait exact) and
  // their rows are never used.
  const int seg = tid % SEGS;
  const int32_t* lsrc = a.W > 0 ? list : a.lengths + li;  // always a valid address
  const bool loader = KPP <= TK || tid / SEGS < TK;  // threads with a key to load
  struct Rows {
    int32_t id[PASSES];
    uint4 k[PASSES], v[PASSES];
    int info[PASSES];
  };
  Rows rows, rows_b;  // rows_b: the second tile of the prologue only
  auto fetch_ids = [&](Rows& r, int tile) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int j = tile * TK + p * KPP + (loader ? tid / SEGS : 0);
      const int jl = j < n_list ? j : (n_list > 0 ? n_list - 1 : 0);
      const int32_t* src = lsrc + jl;
      if (paged) {  // a causal-block key: its slot (one unconditional load either way)
        const int64_t loc = c0 + (j - n_list);
        src = j < n_list ? src : smap.row + (loc < smap.width ? loc : 0);
      }
      r.id[p] = *src;
    }
  };
  auto load_tile = [&](Rows& r, int tile) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int j = tile * TK + p * KPP + (loader ? tid / SEGS : 0);
      const int32_t l = r.id[p];
      const bool in_list = j < n_list;
      const int64_t loc = c0 + (j - n_list);
      const bool valid = in_list ? (unsigned)l < (unsigned)a.Tk
                                 : j < n_tot && (!paged || (loc < smap.width && (unsigned)l < (unsigned)a.Tk));
      const int32_t id = in_list || paged ? l : (int32_t)loc;
      r.info[p] = valid ? (in_list ? -1 : j - n_list) : -2;
      const uint32_t row = valid ? (uint32_t)id : 0u;
      if constexpr (OFF32) {
        // byte offsets fit in 32 bits (checked on the host): base in SGPRs + one VGPR offset
        const uint32_t off = (__umul24(row, (uint32_t)a.kv_st) + seg * 8) * (uint32_t)sizeof(T);
        r.k[p] = *(const uint4*)((const char*)kb + off);
        r.v[p] = *(const uint4*)((const char*)vb + off);
      } else {
        const uint64_t off = (uint64_t)row * (uint64_t)a.kv_st + seg * 8;
        r.k[p] = *(const uint4*)(kb + off);
        r.v[p] = *(const uint4*)(vb + off);
      }
    }
  };
  // Skipped keys store zero rows (their weights are zero; a zero row keeps them so even when
  // the clamped row holds non-finite values): a uniform branch, most tiles have none. A
  // sub-tile holding a key that is not a list key is tagged with the tile number, so the
  // math reads one word to learn whether it must mask.
  auto store_tile = [&](const Rows& r, int buf, int tile) {
    if (!loader) return;
    bool all_ok = true;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) all_ok &= r.info[p] >= -1;
    if (__all(all_ok)) {
#pragma unroll
      for (int p = 0; p < PASSES; ++p) {
        const int kk = p * KPP + tid / SEGS;
        *(uint4*)&sh.k[buf][kk][seg * 8] = r.k[p];
        *(uint4*)&sh.v[buf][kk][seg * 8] = r.v[p];
      }
    } else {
#pragma unroll
      for (int p = 0; p < PASSES; ++p) {
        const int kk = p * KPP + tid / SEGS;
        const bool ok = r.info[p] >= -1;
        *(uint4*)&sh.k[buf][kk][seg * 8] = ok ? r.k[p] : make_uint4(0, 0, 0, 0);
        *(uint4*)&sh.v[buf][kk][seg * 8] = ok ? r.v[p] : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int kk = p * KPP + tid / SEGS;
      if (seg == 0) {
        sh.info[buf][kk] = r.info[p];
        if (r.info[p] != -1) sh.odd[buf][kk / TS] = tile;
      }
    }
  };

  f32x16_t o[DB][QB];
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) o[d][qb][r] = 0.0f;
    }
  }
  float m_run[QB], l_run[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_run[qb] = kNegBig;
    l_run[qb] = 0.0f;
  }

  // S^T = K Q^T of sub-tile `half` of the tile in LDS buffer `buf`: rows = its 32 keys,
  // columns = this wave's query rows (the first sub-tile's; later ones are folded into the
  // previous sub-tile's math).
  auto scores = [&](int buf, int half, f32x16_t (&st)[QB]) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) st[qb][r] = 0.0f;
    }
    // every K operand in flight before the first MFMA (LDS latency paid once)
    op_t ka[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s)
      ka[s] = __builtin_bit_cast(op_t, *(const uint4*)&sh.k[buf][TS * half + ln][16 * s + 8 * hh]);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) st[qb] = M::run(ka[s], qop[qb][s], st[qb]);
    }
  };
  // The weights of one sub-tile from its raw scores s: p = exp2(s * scale - m) per query
  // column, packed in pairs into the 16-bit P^T B operand (accumulator regs 8 s' .. 8 s' + 7
  // are keys 16 s' + {4 hh .. 4 hh + 3, 8 + 4 hh .. 8 + 4 hh + 3}), and their sum in two
  // chains, taken from the packed weights the matrix ops consume.
  auto weights = [&](const f32x16_t (&cur)[QB], uint32_t (&pw)[QB][8], float (&ls)[QB][2]) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      ls[qb][0] = ls[qb][1] = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = fast_exp2(fmaf(cur[qb][r], a.scale_log2, -m_run[qb]));
        const float p1 = fast_exp2(fmaf(cur[qb][r + 1], a.scale_log2, -m_run[qb]));
        pw[qb][r / 2] = M::pack2(p0, p1);
        ls[qb][(r / 2) & 1] = M::sum2(pw[qb][r / 2], ls[qb][(r / 2) & 1]);
      }
    }
  };
  // The running max moves lazily: only when some column's max grows by more than
  // 2^kRescale is the state rescaled, so every weight stays at most 2^kRescale. The weights
  // are first made against the current max; a lane whose sum of 16 weights is below
  // 2^kRescale (the common case) holds no weight that large, so no column of the wave can
  // have grown that much and the max is not needed. Otherwise (some sum reached 2^kRescale,
  // or is not a number) the column maxima are taken and, where a column grew by more than
  // 2^kRescale, the state is rescaled and the weights made again: the same rescales, at
  // the same sub-tiles, as taking the max every time.
  auto settle = [&](const f32x16_t (&cur)[QB], uint32_t (&pw)[QB][8], float (&ls)[QB][2]) {
    bool big = false;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) big |= !(ls[qb][0] + ls[qb][1] < 256.0f);
    static_assert(kRescale == 8.0f, "the sum test is against 2^kRescale");
    if (__any(big)) {
      float mt[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        float mx = cur[qb][0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, cur[qb][r]);
        mt[qb] = fmaxf(mx, lane_xor(mx, 32)) * a.scale_log2;
      }
      bool grow = false;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) grow |= mt[qb] > m_run[qb] + kRescale;
      if (__any(grow)) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const float mn = fmaxf(m_run[qb], mt[qb]);
          const float alpha = fast_exp2(m_run[qb] - mn);
          m_run[qb] = mn;
          l_run[qb] *= alpha;
#pragma unroll
          for (int d = 0; d < DB; ++d) {
#pragma unroll
            for (int r = 0; r < 16; ++r) o[d][qb][r] *= alpha;
          }
        }
        weights(cur, pw, ls);
      }
    }
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) l_run[qb] += ls[qb][0] + ls[qb][1];
  };
  // V^T operands of sub-tile `half` of the tile in buffer `buf`: lane (hh, ln) holds dim
  // 32 d + ln at keys 16 sp + {4 hh .. 4 hh + 3, 8 + 4 hh .. 8 + 4 hh + 3}, two
  // transposing 8-byte reads each.
  constexpr int VROW = 2 * (D + VPAD);  // bytes per V row
  auto v_operands = [&](int buf, int half, op_t (&va)[2][DB]) {
    const lds_char* vbase = (const lds_char*)&sh.v[buf][TS * half][0] + vlane;
#pragma unroll
    for (int sp = 0; sp < 2; ++sp) {
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        const uint2 lo = v_column4(vbase, 16 * sp * VROW + 64 * d);
        const uint2 hi = v_column4(vbase, (16 * sp + 8) * VROW + 64 * d);
        va[sp][d] = __builtin_bit_cast(op_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
      }
    }
  };
  // O^T += V^T P^T for one sub-tile
  auto pv = [&](const op_t (&va)[2][DB], const uint32_t (&pw)[QB][8]) {
#pragma unroll
    for (int sp = 0; sp < 2; ++sp) {
#pragma unroll
      for (int d = 0; d < DB; ++d) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const op_t pb = __builtin_bit_cast(
              op_t, make_uint4(pw[qb][4 * sp], pw[qb][4 * sp + 1], pw[qb][4 * sp + 2], pw[qb][4 * sp + 3]));
          o[d][qb] = M::run(va[sp][d], pb, o[d][qb]);
        }
      }
    }
  };
  // One sub-tile step of a wave, software-pipelined over three sub-tiles so that its matrix
  // and vector work are independent: the weights of sub-tile (cb, ch) (raw scores cur) are
  // made while the matrix core forms the scores of the next sub-tile (nb, nh) into nxt and
  // O^T += V^T P^T of the previous one (buffer pbuf, half ph, weights pwp). One scheduling
  // region (between the issue-priority changes) holds the 16 matrix ops, the exponentials
  // and the pipeline's gathers (hook), none of which depend on each other; the rescale test
  // follows. pre() runs before the region (it may branch). After the last sub-tile the next
  // scores read a stale buffer and are never used.
  auto tile_math = [&](int cb, int ch, int ctile, int nb, int nh, int pbuf, int ph, f32x16_t (&cur)[QB],
                       f32x16_t (&nxt)[QB], uint32_t (&pw)[QB][8], const uint32_t (&pwp)[QB][8], auto&& pre,
                       auto&& hook) {
    // the next sub-tile's K operands and this sub-tile's tag, in flight together
    op_t ka[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s)
      ka[s] = __builtin_bit_cast(op_t, *(const uint4*)&sh.k[nb][TS * nh + ln][16 * s + 8 * hh]);
    // the mask only where the sub-tile holds a skipped or local key (a uniform branch: most
    // sub-tiles are list keys every row sees)
    if (__builtin_amdgcn_readfirstlane(sh.odd[cb][ch]) == ctile) {
      // the lane's 16 keys: 8 (r / 4) + 4 hh + r % 4, four runs of four
      int kinf[16];
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int4 v4 = *(const int4*)&sh.info[cb][TS * ch + 8 * r4 + 4 * hh];
        kinf[4 * r4 + 0] = v4.x; kinf[4 * r4 + 1] = v4.y; kinf[4 * r4 + 2] = v4.z; kinf[4 * r4 + 3] = v4.w;
      }
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int inf = kinf[r];
          const bool vis = (inf == -1) | ((unsigned)inf <= (unsigned)tok[qb]);
          cur[qb][r] = vis ? cur[qb][r] : -INFINITY;
        }
      }
    }
    pre();
    // The two waves of a SIMD alternate between this matrix-heavy region and the rescale
    // test; raising the wave's issue priority here lets its matrix ops issue first.
    __builtin_amdgcn_s_setprio(1);
    op_t va[2][DB];
    v_operands(pbuf, ph, va);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) nxt[qb][r] = 0.0f;
    }
    float ls[QB][2];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) ls[qb][0] = ls[qb][1] = 0.0f;
    // k-step s: the score op s, its share of the weights, the P V op s - 1, then hook(s).
    // The weights are pinned where they are made (an empty asm that uses them): otherwise
    // instruction selection sinks the exponentials to their uses after the last matrix op.
    // The scheduler then interleaves freely: a sched_barrier after each k-step (the source
    // order exactly) measured 6% slower.
    constexpr int EPS = 16 / KS;  // weights per k-step (even)
    constexpr int NPV = 2 * DB;   // P V ops
    auto pv_op = [&](int j) {
      const int sp = j / DB, d = j % DB;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const op_t pb = __builtin_bit_cast(
            op_t, make_uint4(pwp[qb][4 * sp], pwp[qb][4 * sp + 1], pwp[qb][4 * sp + 2], pwp[qb][4 * sp + 3]));
        o[d][qb] = M::run(va[sp][d], pb, o[d][qb]);
      }
    };
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) nxt[qb] = M::run(ka[s], qop[qb][s], nxt[qb]);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
        for (int e = 0; e < EPS; e += 2) {
          const int r = EPS * s + e;
          const float p0 = fast_exp2(fmaf(cur[qb][r], a.scale_log2, -m_run[qb]));
          const float p1 = fast_exp2(fmaf(cur[qb][r + 1], a.scale_log2, -m_run[qb]));
          pw[qb][r / 2] = M::pack2(p0, p1);
          ls[qb][(r / 2) & 1] = M::sum2(pw[qb][r / 2], ls[qb][(r / 2) & 1]);
          asm volatile("" ::"v"(pw[qb][r / 2]));
        }
      }
      if (s >= 1 && s - 1 < NPV) pv_op(s - 1);
      hook(s);
    }
#pragma unroll
    for (int j = KS - 1; j < NPV; ++j) pv_op(j);
    __builtin_amdgcn_s_setprio(0);
    settle(cur, pw, ls);
  };

  // Pipeline, one barrier per tile over NBUF = 4 LDS buffers. Iteration t makes the weights
  // of tile t's two sub-tiles; with them the matrix core forms the scores of the sub-tile
  // after each (tile t's second, tile t + 1's first) and the P V product of the sub-tile
  // before each (tile t - 1's second, tile t's first). Before the first sub-tile's region
  // it stores tile t + 2 (gathered in iteration t - 1); inside the region it gathers tile
  // t + 3 (ids fetched in iteration t - 1), inside the second it fetches the ids of tile
  // t + 4. Iteration t reads buffers t - 1, t and t + 1 (mod 4) and writes buffer t + 2 =
  // t - 2, whose last reads were in iteration t - 1, before the barrier; tile t + 2 is first
  // read after the barrier of iteration t + 1. The vector-memory counter retires in order,
  // and every wait is for the oldest loads outstanding.
  f32x16_t st_a[QB], st_b[QB];
  uint32_t pw_a[QB][8], pw_b[QB][8];
  auto step = [&](int tile) {
    __syncthreads();
    const bool store_next = tile + 2 < n_tiles;
    tile_math(
        tile % NBUF, 0, tile, tile % NBUF, 1, (tile + NBUF - 1) % NBUF, 1, st_a, st_b, pw_a, pw_b,
        [&] {
          if (store_next) store_tile(rows, (tile + 2) % NBUF, tile + 2);
        },
        [&](int s) {
          if (s == 3) load_tile(rows, tile + 3);
        });
    tile_math(
        tile % NBUF, 1, tile, (tile + 1) % NBUF, 0, tile % NBUF, 0, st_b, st_a, pw_b, pw_a, [] {},
        [&](int s) {
          if (s == 1) fetch_ids(rows, tile + 4);
        });
  };
  fetch_ids(rows, 0);
  fetch_ids(rows_b, 1);
  load_tile(rows, 0);
  load_tile(rows_b, 1);
  // the first sub-tile has no previous one: its P V product takes zero weights and the
  // second half of buffer NBUF - 1, zeroed here (tile 3 is first stored there in iteration 1)
  {
    uint4* z = (uint4*)&sh.v[NBUF - 1][TS][0];  // rows TS .. TK - 1, contiguous
    for (int x = tid; x < TS * (D + VPAD) / 8; x += NTH) z[x] = make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
    for (int j = 0; j < 8; ++j) pw_b[qb][j] = 0u;
  }
  store_tile(rows, 0, 0);
  fetch_ids(rows, 2);
  store_tile(rows_b, 1, 1);
  load_tile(rows, 2);
  fetch_ids(rows, 3);
  __syncthreads();
  scores(0, 0, st_a);
  for (int tile = 0; tile < n_tiles; ++tile) step(tile);
  // the last sub-tile's P V product
  {
    op_t va[2][DB];
    v_operands((n_tiles - 1) % NBUF, 1, va);
    pv(va, pw_b);
  }

  // normalise and store: lane (hh, q) holds dims 32 d + 8 (r / 4) + 4 hh + r % 4 of column q
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float lt = l_run[qb] + lane_xor(l_run[qb], 32);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    if (!qok[qb]) continue;
    T* op = (T*)a.out + qrow[qb];
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int dim = 32 * d + 8 * r4 + 4 * hh;
        uint2 u;
        u.x = M::pack2(o[d][qb][4 * r4 + 0] * inv, o[d][qb][4 * r4 + 1] * inv);
        u.y = M::pack2(o[d][qb][4 * r4 + 2] * inv, o[d][qb][4 * r4 + 3] * inv);
        *(uint2*)(op + dim) = u;
      }
    }
  }
}

constexpr int kQB = 1;  // one block of 32 query columns per wave (two waves a SIMD)

template <typename T, bool OFF32>
void launch_prefill(const PrefillArgs& a, int D, dim3 grid, hipStream_t s) {
  constexpr int nth = 64 * (8 / kQB);
  if (D == 64) prefill_mfma_kernel<T, 64, kQB, OFF32><<<grid, nth, 0, s>>>(a);
  else prefill_mfma_kernel<T, 128, kQB, OFF32><<<grid, nth, 0, s>>>(a);
}

}  // namespace

// Whether the MFMA tile kernel serves a chunked read of this shape: 16-bit rows, head dim
// 64 or 128, chunk in {16, 32, 64, 128, 256} (a workgroup holds 256 query rows).
extern "C" int lsa_read_chunked_mfma_ok(int dtype, int32_t D, int32_t chunk) {
  const bool type_ok = dtype == LSA_BF16 || dtype == LSA_F16;
  const bool d_ok = D == 64 || D == 128;
  const bool c_ok = chunk == 16 || chunk == 32 || chunk == 64 || chunk == 128 || chunk == 256;
  return (type_ok && d_ok && c_ok) ? 1 : 0;
}

namespace lsa {

// Launches the MFMA chunked read (arguments already checked by lsa_read_chunked).
int launch_read_chunked_mfma(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t T, int64_t Tk,
                             int32_t Hq, int32_t Hkv, int32_t D, int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                             const int32_t* ids, const int32_t* lengths, int32_t W, int32_t chunk,
                             const SlotMap& slots, float scale, void* out, hipStream_t s) {
  PrefillArgs a;
  a.slots = slots;
  a.q = q; a.k = k; a.v = v; a.out = out; a.ids = ids; a.lengths = lengths;
  a.T = T; a.Tk = Tk; a.kv_sb = kv_sb; a.kv_st = kv_st; a.kv_sh = kv_sh;
  a.Hq = Hq; a.Hkv = Hkv; a.W = W; a.chunk = chunk;
  a.C = (int)((T + chunk - 1) / chunk);
  const int gq = Hq / Hkv;
  const int per = kRows / chunk;  // heads that fill the workgroup's rows
  a.hpw = per < gq ? per : gq;
  a.n_hg = (gq + a.hpw - 1) / a.hpw;
  a.scale_log2 = scale * kLog2e;
  const int64_t n = B * a.C * Hkv * a.n_hg;
  LSA_REQUIRE(n <= 0x7FFFFFFF, LSA_ERR_SHAPE, "lsa_read_chunked: too many workgroups");
  if (n == 0) return LSA_OK;
  // 32-bit gather offsets when every row of one (batch, kv-head) view is within 4 GiB of its
  // first and the row index and stride fit the 24-bit multiply
  const uint64_t span = (uint64_t)(Tk > 0 ? Tk - 1 : 0) * (uint64_t)kv_st * 2u + (uint64_t)D * 2u;
  const bool off32 = span < (1ull << 32) && Tk < (1 << 24) && kv_st < (1 << 24);
  const dim3 grid((unsigned)n);
  if (dtype == LSA_BF16) {
    if (off32) launch_prefill<bf16_t, true>(a, D, grid, s);
    else launch_prefill<bf16_t, false>(a, D, grid, s);
  } else {
    if (off32) launch_prefill<_Float16, true>(a, D, grid, s);
    else launch_prefill<_Float16, false>(a, D, grid, s);
  }
  LSA_LAUNCHED("lsa_read_chunked (mfma)");
  return LSA_OK;
}

}  // namespace lsa
