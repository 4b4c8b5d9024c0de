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
#include "lsa_read_dev.h"

using namespace lsa;

namespace lsa {
int launch_read_chunked_mfma(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t T, int64_t Tk,
                             int32_t Hq, int32_t Hkv, int32_t D, int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                             const int32_t* ids, const int32_t* lengths, int32_t W, int32_t chunk,
                             const SlotMap& slots, float scale, void* out, hipStream_t s);
}  // namespace lsa

namespace {

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
  SlotMap slots;  // chunked reads of a paged cache: the causal block's positions -> cache rows
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
  SlotRow map;  // the causal block's positions -> cache rows (identity without a slot table)
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
    r.map = slot_row_of(a.slots, b);
  } else {
    const int64_t li = a.ids_per_head ? row * a.Hkv + g : row;
    int n = a.lengths[li];
    n = (n < 0 || a.Tk <= 0) ? 0 : (n > a.W ? a.W : n);
    r.ids = a.ids + li * a.W;
    r.n_list = n;
    r.local_start = 0;
    r.n = n;
    r.map = SlotRow{nullptr, 0};
  }
  return r;
}

// Token id of list slot j (< hi), or -1; the ids load is unconditional (clamped slot).
__device__ __forceinline__ int32_t slot_id(const RowList& l, int j, int hi) {
  const int jl = j < l.n_list ? j : (l.n_list > 0 ? l.n_list - 1 : 0);
  const int32_t x = l.n_list > 0 ? l.ids[jl] : -1;
  int32_t local = (int32_t)(l.local_start + (j - l.n_list));
  if (l.map.row != nullptr) {  // a paged cache (uniform branch): the slot table, loaded unconditionally
    const bool in = local >= 0 && local < l.map.width;
    const int32_t m = l.map.row[in ? local : 0];
    local = in ? m : -1;
  }
  return j >= hi ? -1 : (j < l.n_list ? x : local);
}

template <typename T, int D, int GQ>
__global__ __launch_bounds__(LSA_BLOCK) void read_kernel(ReadArgs a) {
  using S = ReadShape<T, D, GQ>;
  constexpr int VEC = S::VEC, LPT = S::LPT;
  constexpr int PSTRIDE = GQ * (D + 2);  // floats per partial
  __shared__ ReadLds<D, GQ, kMaxSplits> sh;

  const int64_t i = blockIdx.x;
  const int s = blockIdx.y;
  const int64_t row = i / a.Hkv;
  const int g = (int)(i % a.Hkv);
  const int lp = (threadIdx.x & (LSA_WAVE - 1)) % LPT;

  const RowList list = row_list(a, row, g);
  const int n_act = (list.n + a.span - 1) / a.span;
  if (s >= (n_act > 0 ? n_act : 1)) return;  // idle split
  T* outp = (T*)a.out + (row * a.Hq + (int64_t)g * GQ) * D;
  if (list.n == 0) {  // nothing to read: zeros (tiled contract) or NaN (v1 contract)
    for (int j = threadIdx.x; j < GQ * D; j += LSA_BLOCK) store_out<T>(outp + j, a.empty_nan ? NAN : 0.0f);
    return;
  }
  const int lo = s * a.span;
  const int hi = min(lo + a.span, list.n);
  const int64_t b = row / a.Tq;
  const T* kb = (const T*)a.k + b * a.kv_sb + g * a.kv_sh + lp * VEC;
  const T* vb = (const T*)a.v + b * a.kv_sb + g * a.kv_sh + lp * VEC;
  const T* qrow = (const T*)a.q + (row * a.Hq + (int64_t)g * GQ) * D;

  AttnState<T, D, GQ> st;
  attend_span<T, D, GQ>(qrow, kb, vb, a.kv_st, a.Tk, lo, hi, [&](int j) { return slot_id(list, j, hi); },
                        a.scale_log2, st);
  float* part = n_act > 1 ? a.ws_part + (i * (int64_t)gridDim.y + s) * PSTRIDE : nullptr;
  finish_span<T, D, GQ, kMaxSplits, true>(sh, st, n_act == 1, outp, part, a.empty_nan);
  if (n_act == 1) return;
  if (!arrive_last(&a.ws_count[i], n_act, &sh.flag)) return;
  combine_partials<T, D, GQ>(sh, a.ws_part + i * (int64_t)gridDim.y * PSTRIDE, n_act, outp, a.empty_nan);
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
  a.slots = SlotMap{nullptr, nullptr, 0, 0, 0};
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
                                const int32_t* lengths, int32_t W, int32_t chunk, const lsa_slot_map* slots,
                                float scale, int32_t path, void* out, void* stream) {
  int rc = check_read_common(q, k, v, dtype, B, T, Tk, Hq, Hkv, D, kv_batch_stride, kv_token_stride,
                             kv_head_stride, ids, lengths, W, out);
  if (rc != LSA_OK) return rc;
  SlotMap sm;
  LSA_TRY(check_slots("lsa_read_chunked", slots, &sm));
  LSA_REQUIRE(chunk >= 1, LSA_ERR_SHAPE, "lsa_read_chunked: chunk must be >= 1");
  // positions are cache rows unless the cache is paged (then the slot table maps them)
  LSA_REQUIRE(slots || T <= Tk, LSA_ERR_SHAPE, "lsa_read_chunked: %lld query rows exceed the cache %lld",
              (long long)T, (long long)Tk);
  LSA_REQUIRE(B * T * Hkv <= 0x7FFFFFFF, LSA_ERR_SHAPE, "lsa_read_chunked: too many rows");
  LSA_REQUIRE(path >= LSA_CHUNKED_AUTO && path <= LSA_CHUNKED_MFMA, LSA_ERR_SHAPE, "lsa_read_chunked: path %d", path);
  const int mfma_ok = lsa_read_chunked_mfma_ok(dtype, D, chunk);
  LSA_REQUIRE(path != LSA_CHUNKED_MFMA || mfma_ok, LSA_ERR_SHAPE,
              "lsa_read_chunked: the MFMA path needs bf16/fp16 rows, D 64/128 and a power-of-two chunk 16..256");
  if (B * T * Hkv == 0) return LSA_OK;
  if (mfma_ok && path != LSA_CHUNKED_GATHER)
    return launch_read_chunked_mfma(q, k, v, dtype, B, T, Tk, Hq, Hkv, D, kv_batch_stride, kv_token_stride,
                                    kv_head_stride, ids, lengths, W, chunk, sm, scale, out, (hipStream_t)stream);
  ReadArgs a;
  a.q = q; a.k = k; a.v = v; a.out = out; a.ids = ids; a.lengths = lengths;
  a.Tq = T; a.Tk = Tk; a.Hq = Hq; a.Hkv = Hkv; a.W = W; a.ids_per_head = 1; a.chunk = chunk; a.slots = sm;
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
