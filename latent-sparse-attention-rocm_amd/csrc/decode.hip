// Fused decode step for gfx950: group-mean index queries, flat select and the split sparse
// read in one launch (reference port/bench.py:147-153, the decode step = flat_select then
// the sparse read; pipeline.py:248-316, select_fused.py:52-280, read_kernel_tiled.py:92-156).
//
// A unit is one (query row, kv-head). The 1-D grid holds the select workgroups of every
// unit first, then the readers.
//
// Select workgroup (unit i, split s), id s * units + i: the unit's index query is the fp32
// mean of its query group's rows (summed in head order, divided by the group size, as the
// separate index-query kernel does); it scores columns [s*cs, (s+1)*cs) of the unit's
// bucket table (the canonical score), publishes the keys and arrives. The last split of a
// unit takes every key, selects the K best buckets in rank order, counts each picked
// bucket's kept members (sink <= id < window start, in table order) and publishes the
// unit's record: per pick, word A = bucket + 2 and word B = end of the pick's slots in the
// list (the clipped inclusive prefix of kept counts) + 1. Both words are nonzero once
// written, so a reader that sees all 2K words nonzero holds the whole record: no flag and
// no fence. It also writes the unit's list length.
//
// Rank form (tables of at most kRankMaxRows buckets, more than one split, the published
// keys fit the counters region): no split collects. Each split publishes its columns' keys
// + 1 (nonzero once written) into the counters region and exits; every reader of the unit
// waits until all of the unit's keys are nonzero, ranks them itself (the same top-K on the
// same keys), takes each pick's kept count from the span ends it loaded while waiting (or
// from the picks' member rows), and reads its share. Role 0 writes the list length; the last reader to arrive
// zeroes the published keys. This drops the last split's arrival, its reload of the keys,
// the record and its poll from the step's chain.
//
// Reader workgroup (unit i, pick j, part u) or (unit i, tail part t): waits for the record
// with a bounded poll (past the limit it sets *status and exits), expands its share of the
// list - the kept members of pick j at ranks [u*span, u*span + span), or a slice of the
// window-then-sinks tail - into LDS and into the list, gathers those K/V rows and publishes
// a split partial (or writes the output when the unit has one active part). Every reader
// of the unit then arrives; the last one combines the partials, clears the record and
// resets the counter, so the workspace is ready for the next launch.
//
// Readers wait only on select workgroups, which hold lower ids. Workgroups are dispatched
// in id order, so every select workgroup is resident (or done) before any reader can
// occupy a slot, and it never waits itself: the readers' wait ends.
#include "lsa_abi_common.h"
#include "decode_dev.h"

using namespace lsa;
using namespace lsa::decode;

namespace {

// ------------------------------------------------------------------ host

struct Plan {
  bool rep;         // replicated select: every workgroup is a reader that selects for itself
  int K, kp, span, NR;
  int64_t cstride;  // words between record copies
  size_t keys_bytes, part_bytes, shmem;
};

template <int D, int GQ>
size_t reader_lds(int span) {
  return rd_ids_offset<D, GQ>() + sizeof(int32_t) * (size_t)kChunkTiles * span;
}

template <int D>
size_t reader_lds_gq(int gq, int span) {
  switch (gq) {
    case 1: return reader_lds<D, 1>(span);
    case 2: return reader_lds<D, 2>(span);
    case 4: return reader_lds<D, 4>(span);
    default: return reader_lds<D, 8>(span);
  }
}

size_t reader_lds_d(int D, int gq, int span) {
  switch (D) {
    case 32: return reader_lds_gq<32>(gq, span);
    case 64: return reader_lds_gq<64>(gq, span);
    case 128: return reader_lds_gq<128>(gq, span);
    default: return reader_lds_gq<256>(gq, span);
  }
}

template <int D>
size_t rank_lds_gq(int gq, int rows) {
  switch (gq) {
    case 1: return rank_lds<D, 1>(rows);
    case 2: return rank_lds<D, 2>(rows);
    case 4: return rank_lds<D, 4>(rows);
    default: return rank_lds<D, 8>(rows);
  }
}

size_t rank_lds_d(int D, int gq, int rows) {
  switch (D) {
    case 32: return rank_lds_gq<32>(gq, rows);
    case 64: return rank_lds_gq<64>(gq, rows);
    case 128: return rank_lds_gq<128>(gq, rows);
    default: return rank_lds_gq<256>(gq, rows);
  }
}

template <int D>
size_t rep_lds_gq(int gq, int span) {
  switch (gq) {
    case 1: return rep_ids_offset<D, 1>() + sizeof(int32_t) * (size_t)kRepChunkTiles * span;
    case 2: return rep_ids_offset<D, 2>() + sizeof(int32_t) * (size_t)kRepChunkTiles * span;
    case 4: return rep_ids_offset<D, 4>() + sizeof(int32_t) * (size_t)kRepChunkTiles * span;
    default: return rep_ids_offset<D, 8>() + sizeof(int32_t) * (size_t)kRepChunkTiles * span;
  }
}

// LDS of a replicated-select workgroup; 0 where that kernel does not exist (D = 256).
size_t rep_lds_d(int D, int gq, int span) {
  switch (D) {
    case 32: return rep_lds_gq<32>(gq, span);
    case 64: return rep_lds_gq<64>(gq, span);
    case 128: return rep_lds_gq<128>(gq, span);
    default: return 0;
  }
}

// Why the replicated select cannot serve a shape (nullptr: it can).
const char* rep_unfit(int dtype, int D, int gq, int rows, int top_p, int score_mode, int table_flags) {
  if (!(table_flags & LSA_TABLE_SPANS)) return "it needs span tables (LSA_TABLE_SPANS)";
  if (table_flags & LSA_TABLE_BLOCK_VISIBLE) return "it takes visibility from the span ends";
  if (score_mode != LSA_SCORE_BF16) return "it scores bf16 centroids only";
  if (D > 128) return "head dim above 128";
  if (rows > kRepMaxRows) return "more buckets than it holds in LDS";
  if ((top_p < rows ? top_p : rows) > kMaxPicks) return "more than 64 picks";
  const int span = lsa_read_tile_tokens(dtype, D, gq);
  if (span <= 0 || rep_lds_d(D, gq, span) + 4096 > kMaxLds) return "its LDS exceeds 64 KiB";
  return nullptr;
}

// Record copies sit one 4 KiB page plus 256 bytes apart, so readers polling different
// copies load from different memory channels.
int64_t record_stride(int64_t units, int K) {
  const int64_t words = units * 2 * K;
  return ((words + 1023) / 1024) * 1024 + 64;
}

// Readers per unit: with few units, about one tile of the list a reader (picks are buckets
// of ~one tile, plus the tail's tiles), so the gather spreads over as many CUs as it can
// use, but at most kDefaultMaxReaders: past ~24 a unit, the wider combine and the extra
// workgroups' launch cost more than the shorter gathers save (32k decode, B=1, rank form
// with 32 select splits: 18.4 us with 24 readers, 18.6 with 16, 19.1 with 32, 20.4 with
// 40; the record form: 22.5 us with 32, 21.2 with 16 or 24); with many units, enough
// readers for ~512 workgroups in all, each streaming a run of tiles through the pipelined
// gather (B=32 x 32k flat: 82.8 us with 2 readers a unit, 88.4 with 3, 83.5 with 4, 85.6
// with 6; the B=32 x 131k tree: 76.9 / 83.9 / 78.5 / 81.0).
constexpr int kDefaultMaxReaders = 24;
constexpr int kReaderSpread = 512;

int default_readers(int64_t units, int K, int span, int window, int sink) {
  const int64_t tail = ((int64_t)window + sink + span - 1) / span;
  int64_t nr = (int64_t)K + tail;
  const int64_t spread = (kReaderSpread + units - 1) / units;
  if (spread < nr) nr = spread;
  if (nr > kDefaultMaxReaders) nr = kDefaultMaxReaders;
  if (nr < 1) nr = 1;
  return (int)(nr < kMaxReaders ? nr : kMaxReaders);
}

int plan_decode(int dtype, int D, int gq, int64_t units, int rows, int top_p, int window, int sink, int splits,
                int readers, Plan* p) {
  p->rep = splits == 0;
  p->K = top_p < rows ? top_p : rows;
  p->kp = next_pow2(p->K);
  p->span = lsa_read_tile_tokens(dtype, D, gq);
  LSA_REQUIRE(p->span > 0, LSA_ERR_SHAPE, "lsa_decode_flat: no read tile for D=%d group=%d", D, gq);
  LSA_REQUIRE(readers >= 0 && readers <= kMaxReaders, LSA_ERR_SHAPE, "lsa_decode_flat: readers in [0, %d], got %d",
              kMaxReaders, readers);
  p->NR = readers > 0 ? readers : default_readers(units, p->K, p->span, window, sink);
  p->cstride = record_stride(units, p->K);
  p->keys_bytes = splits > 1 ? (size_t)units * rows * sizeof(uint64_t) : 0;
  p->part_bytes = p->NR > 1 ? (size_t)units * p->NR * (size_t)(gq * (D + 2)) * sizeof(float) : 0;
  if (p->rep) {
    p->keys_bytes = 0;
    p->shmem = rep_lds_d(D, gq, p->span);
    return LSA_OK;
  }
  size_t sel = sel_keys_offset() + sizeof(uint64_t) * ((size_t)rows + p->kp);
  const size_t scr = sel_keys_offset() + sizeof(ScreenLds) + sizeof(uint64_t) * (size_t)p->kp;
  if (splits == 1 && scr > sel) sel = scr;  // a lone split may screen its table (screen_topk)
  const size_t rd = reader_lds_d(D, gq, p->span);
  p->shmem = sel > rd ? sel : rd;
  return LSA_OK;
}

}  // namespace

extern "C" int lsa_decode_flat_rep_ok(int dtype, int32_t D, int32_t group, int32_t rows, int32_t top_p,
                                      int score_mode, int32_t table_flags) {
  if (!(D == 32 || D == 64 || D == 128) || !(group == 1 || group == 2 || group == 4 || group == 8)) return 0;
  if (rows < 1 || top_p < 1) return 0;
  return rep_unfit(dtype, D, group, rows, top_p, score_mode, table_flags) == nullptr ? 1 : 0;
}

// Word offset of the rank form's published keys in the counters region (after the arrival
// counters and the record copies, 256-byte aligned), and whether a table shape has them.
int64_t rank_keys_at(int64_t units, int K) {
  return ((2 * units + kRecordCopies * record_stride(units, K)) + 63) / 64 * 64;
}
bool rank_slots(int64_t units, int rows) { return rows <= kRankMaxRows && units * rows <= kRankMaxSlots; }

extern "C" int64_t lsa_decode_flat_counters(int64_t R, int32_t Hkv, int32_t rows, int32_t top_p) {
  if (R <= 0 || Hkv <= 0 || rows <= 0 || top_p <= 0) return 0;
  const int K = top_p < rows ? top_p : rows;
  if (K > kMaxPicks) return 0;
  const int64_t units = R * Hkv;
  if (rank_slots(units, rows)) return rank_keys_at(units, K) + 2 * units * rows;
  return 2 * units + kRecordCopies * record_stride(units, K);
}

extern "C" size_t lsa_decode_flat_scratch_bytes(int dtype, int64_t R, int32_t Hq, int32_t Hkv, int32_t D,
                                                int32_t rows, int32_t top_p, int32_t window, int32_t sink,
                                                int32_t select_splits, int32_t readers) {
  if (R <= 0 || Hkv <= 0 || Hq < Hkv || rows <= 0 || top_p <= 0) return 0;
  Plan p;
  if (plan_decode(dtype, D, Hq / Hkv, R * Hkv, rows, top_p, window < 0 ? 0 : window, sink < 0 ? 0 : sink,
                  select_splits, readers, &p) != LSA_OK)
    return 0;
  return ((p.keys_bytes + 255) & ~(size_t)255) + p.part_bytes;
}

namespace {

// A one-level node tree for the fused decode's select (lsa_decode_tree).
struct TreeSpec {
  const void* node_centroids;
  const int32_t* children;
  int32_t n_nodes, node_size, node_block, beam_width;
};

int decode_launch(const char* who, const void* q, const void* k, const void* v, int dtype, int64_t R, int64_t Tk,
                  int32_t Hq, int32_t Hkv, int32_t D, int64_t kv_batch_stride, int64_t kv_token_stride,
                  int64_t kv_head_stride, const void* centroids, const int32_t* members, const int32_t* ends,
                  int32_t table_flags, int32_t rows, int32_t cap, int64_t row_tables, int64_t group_tables,
                  int score_mode, const int32_t* positions, const lsa_slot_map* slots, int32_t cluster_block_size,
                  int32_t block_buckets, int32_t top_p, int32_t window, int32_t sink, int32_t top_k, float scale,
                  int32_t select_splits, int32_t readers, int32_t* counters, int64_t n_counters, void* scratch,
                  size_t scratch_bytes, int32_t* lists, int32_t* lengths, void* out, int32_t* status, void* stream,
                  const TreeSpec* tree) {
  LSA_REQUIRE(q && k && v && centroids && members && positions && lists && lengths && out && counters, LSA_ERR_NULL,
              "%s: NULL pointer", who);
  SlotMap sm;
  LSA_TRY(check_slots(who, slots, &sm));
  LSA_REQUIRE(dtype == LSA_F32 || dtype == LSA_BF16 || dtype == LSA_F16, LSA_ERR_DTYPE,
              "%s: dtype %d", who, dtype);
  LSA_REQUIRE(D == 32 || D == 64 || D == 128 || D == 256, LSA_ERR_SHAPE,
              "%s: head dim %d not in {32,64,128,256}", who, D);
  LSA_REQUIRE(Hq >= 1 && Hkv >= 1 && Hq % Hkv == 0, LSA_ERR_SHAPE, "%s: Hq %d must group onto Hkv %d", who,
              Hq, Hkv);
  const int gq = Hq / Hkv;
  LSA_REQUIRE(gq == 1 || gq == 2 || gq == 4 || gq == 8, LSA_ERR_SHAPE,
              "%s: group size %d not in {1,2,4,8}", who, gq);
  LSA_REQUIRE(score_mode == LSA_SCORE_BF16 || score_mode == LSA_SCORE_F32, LSA_ERR_DTYPE,
              "%s: bad score mode", who);
  LSA_REQUIRE(rows >= 1 && cap >= 1 && row_tables >= 0 && group_tables >= 0, LSA_ERR_SHAPE,
              "%s: bad table sizes", who);
  LSA_REQUIRE(R >= 0 && Tk >= 0 && Tk <= 0x7FFFFFFF, LSA_ERR_SHAPE, "%s: bad sizes", who);
  LSA_REQUIRE(top_p >= 1 && window >= 0 && sink >= 0 && top_k >= 0, LSA_ERR_SHAPE,
              "%s: top_p >= 1, window/sink/top_k >= 0", who);
  LSA_REQUIRE(ends || cluster_block_size >= 1, LSA_ERR_SHAPE, "%s: cluster_block_size must be >= 1", who);
  LSA_REQUIRE((table_flags & ~(LSA_TABLE_SPANS | LSA_TABLE_BLOCK_VISIBLE)) == 0, LSA_ERR_SHAPE,
              "%s: unknown table flags %d", who, table_flags);
  LSA_REQUIRE(!(table_flags & LSA_TABLE_BLOCK_VISIBLE) || cluster_block_size >= 1, LSA_ERR_SHAPE,
              "%s: cluster_block_size must be >= 1", who);
  LSA_REQUIRE(!(table_flags & LSA_TABLE_SPANS) || ends, LSA_ERR_SHAPE,
              "%s: LSA_TABLE_SPANS needs the span ends", who);
  const int K = top_p < rows ? top_p : rows;
  LSA_REQUIRE(K <= kMaxPicks, LSA_ERR_SHAPE, "%s: %d picks exceed %d", who, K, kMaxPicks);
  LSA_REQUIRE((int64_t)K * cap < 0x7FFFFFFF && (int64_t)top_k + window + sink <= 0x7FFFFFFF, LSA_ERR_SHAPE,
              "%s: list too wide", who);
  LSA_REQUIRE(select_splits >= 0 && select_splits <= 256 && select_splits <= rows, LSA_ERR_SHAPE,
              "%s: select splits in [0, min(256, rows)], got %d", who, select_splits);
  if (select_splits == 0) {
    const char* why = rep_unfit(dtype, D, gq, rows, top_p, score_mode, table_flags);
    LSA_REQUIRE(why == nullptr, LSA_ERR_SHAPE, "%s: the replicated select (splits 0) does not apply: %s", who,
                why ? why : "");
  }
  const uintptr_t mis = ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)centroids) & 15;
  LSA_REQUIRE(mis == 0, LSA_ERR_ALIGN, "%s: q/k/v/centroids must be 16-byte aligned", who);
  const int64_t esize = dtype == LSA_F32 ? 4 : 2;
  LSA_REQUIRE(kv_batch_stride >= 0 && kv_token_stride >= D && kv_head_stride >= D, LSA_ERR_SHAPE,
              "%s: K/V strides must leave rows of %d elements apart", who, D);
  LSA_REQUIRE(((kv_batch_stride | kv_token_stride | kv_head_stride) * esize) % 16 == 0, LSA_ERR_ALIGN,
              "%s: K/V strides must keep rows 16-byte aligned", who);
  const int64_t units = R * Hkv;
  if (units == 0) return LSA_OK;
  Plan p;
  LSA_TRY(plan_decode(dtype, D, gq, units, rows, top_p, window, sink, select_splits, readers, &p));
  LSA_REQUIRE(p.rep || p.kp + rows <= 6144, LSA_ERR_SHAPE,
              "%s: %d columns + %d picks exceed 6144 LDS keys", who, rows, p.kp);
  int nodes_pow2 = 0, beam_pow2 = 0, cand_pow2 = 0, top_pow2 = 0;
  bool tree_stash = false, tree_kids4 = false;
  if (tree) {
    LSA_REQUIRE(tree->node_centroids && tree->children, LSA_ERR_NULL, "%s: NULL node tables", who);
    LSA_REQUIRE(tree->n_nodes >= 1 && tree->node_size >= 1 && tree->node_block >= 1 && tree->beam_width >= 1,
                LSA_ERR_SHAPE, "%s: n_nodes, node_size, node_block, beam_width >= 1", who);
    LSA_REQUIRE(rows <= 8192, LSA_ERR_SHAPE, "%s: %d buckets exceed the 8192 of the dedup bitmap", who, rows);
    LSA_REQUIRE((((uintptr_t)tree->node_centroids) & 15) == 0, LSA_ERR_ALIGN,
                "%s: node centroids must be 16-byte aligned", who);
    const int beam = tree->beam_width < tree->n_nodes ? tree->beam_width : tree->n_nodes;
    // fresh buckets [covered, visible): fewer than node_block past the made nodes, or every
    // bucket past the nodes' reach
    const int64_t reach = (int64_t)tree->n_nodes * tree->node_size;
    const int64_t max_fresh = rows - reach > (int64_t)tree->node_block - 1 ? rows - reach : tree->node_block - 1;
    const int64_t cand_cap = (int64_t)beam * tree->node_size + (max_fresh < rows ? max_fresh : rows);
    LSA_REQUIRE(tree->n_nodes <= 6144 && cand_cap <= 6144, LSA_ERR_SHAPE,
                "%s: %d nodes / %lld candidates exceed 6144 LDS keys", who, tree->n_nodes, (long long)cand_cap);
    nodes_pow2 = next_pow2(tree->n_nodes);
    beam_pow2 = next_pow2(beam);
    cand_pow2 = next_pow2((int)(cand_cap > 0 ? cand_cap : 1));
    top_pow2 = next_pow2(p.K < cand_pow2 ? p.K : cand_pow2);
    size_t sel = sel_keys_offset() + sizeof(uint64_t) * (size_t)((nodes_pow2 > cand_pow2 ? nodes_pow2 : cand_pow2) +
                                                                (beam_pow2 > top_pow2 ? beam_pow2 : top_pow2)) +
                 sizeof(int32_t) * (size_t)cand_pow2 + sizeof(uint32_t) * (size_t)((rows + 31) / 32);
    // the children table and span ends staged in LDS with the first round trip, when they fit
    const int64_t words = (int64_t)tree->n_nodes * tree->node_size;
    const size_t stash_end = tree_stash_offset(nodes_pow2, cand_pow2, beam_pow2, top_pow2, rows) +
                             tree_stash_bytes((int)(words < (1 << 24) ? words : (1 << 24)), rows);
    tree_stash = words < (1 << 24) && stash_end <= kMaxLds;
    if (tree_stash) sel = stash_end;
    tree_kids4 = words % 4 == 0 && (((uintptr_t)tree->children) & 15) == 0;
    const size_t rd = reader_lds_d(D, gq, p.span);
    p.shmem = sel > rd ? sel : rd;
  }
  // the rank form: more than one select split over a table whose keys fit the readers and
  // the counters region (which then holds the published keys)
  const bool rank = !tree && !p.rep && select_splits > 1 && rank_slots(units, rows) &&
                    rank_lds_d(D, gq, rows) <= kMaxLds;
  if (rank && rank_lds_d(D, gq, rows) > p.shmem) p.shmem = rank_lds_d(D, gq, rows);
  LSA_REQUIRE(p.shmem <= kMaxLds, LSA_ERR_SHAPE, "%s: %zu bytes of LDS exceed %zu", who, p.shmem, kMaxLds);
  const int64_t grid = units * (select_splits + p.NR);
  LSA_REQUIRE(grid <= 0x7FFFFFFF, LSA_ERR_SHAPE, "%s: too many workgroups", who);
  const int64_t need_counters = lsa_decode_flat_counters(R, Hkv, rows, top_p);
  LSA_REQUIRE(need_counters > 0 && n_counters >= need_counters, LSA_ERR_WORKSPACE,
              "%s: %lld counters < %lld", who, (long long)n_counters, (long long)need_counters);
  const size_t keys_at = (p.keys_bytes + 255) & ~(size_t)255;
  const size_t need = keys_at + p.part_bytes;
  LSA_REQUIRE(need == 0 || (scratch && scratch_bytes >= need), LSA_ERR_WORKSPACE,
              "%s: scratch %zu < %zu bytes", who, scratch_bytes, need);
  LSA_REQUIRE(((uintptr_t)scratch % 16) == 0, LSA_ERR_ALIGN, "%s: scratch must be 16-byte aligned", who);

  DecodeArgs a;
  a.q = q; a.k = k; a.v = v; a.out = out;
  a.R = R; a.G = Hkv; a.Hq = Hq;
  a.Tk = Tk; a.kv_sb = kv_batch_stride; a.kv_st = kv_token_stride; a.kv_sh = kv_head_stride;
  a.centroids = centroids; a.members = members; a.ends = ends; a.rows = rows; a.cap = cap;
  a.vends = (table_flags & LSA_TABLE_BLOCK_VISIBLE) ? nullptr : ends;
  a.vec_rows = (cap % 4 == 0 && ((uintptr_t)members % 16) == 0) ? 1 : 0;
  a.spans = (table_flags & LSA_TABLE_SPANS) ? 1 : 0;
  a.row_tables = row_tables; a.group_tables = group_tables; a.positions = positions;
  a.cluster_block = cluster_block_size; a.block_buckets = block_buckets;
  a.K = p.K; a.kp = p.kp; a.window = window; a.sink = sink; a.top_k = top_k; a.W = top_k + window + sink;
  a.S = select_splits; a.cs = select_splits > 0 ? (rows + select_splits - 1) / select_splits : rows;
  a.screen = select_splits == 1 && score_mode == LSA_SCORE_BF16 && screen_pays(D, rows, p.K) ? 1 : 0;
  a.span = p.span; a.NR = p.NR;
  a.chunk = p.rep ? kRepChunkTiles : kChunkTiles;
  a.tree = tree ? 1 : 0;
  a.node_centroids = tree ? tree->node_centroids : nullptr;
  a.children = tree ? tree->children : nullptr;
  a.n_nodes = tree ? tree->n_nodes : 0;
  a.node_size = tree ? tree->node_size : 0;
  a.node_block = tree ? tree->node_block : 0;
  a.beam = tree ? tree->beam_width : 0;
  a.nodes_pow2 = nodes_pow2; a.beam_pow2 = beam_pow2; a.cand_pow2 = cand_pow2; a.top_pow2 = top_pow2;
  a.ends4 = (ends && rows % 4 == 0 && ((uintptr_t)ends % 16) == 0) ? 1 : 0;
  if (tree) a.screen = 0;
  a.stash = tree_stash ? 1 : 0;
  a.kids4 = tree_kids4 ? 1 : 0;
  a.scale_log2 = scale * kLog2e;
  a.spin_limit = decode_debug().spin_limit > 0 ? decode_debug().spin_limit
                                              : 1 << 22;  // polls of about a microsecond each: seconds
  a.skip_publish = decode_debug().skip_publish;
  a.rank = rank ? 1 : 0;
  a.pub = rank ? (uint64_t*)(counters + rank_keys_at(units, p.K)) : nullptr;
  a.sel_count = counters;
  a.rd_count = counters + units;
  a.record = counters + 2 * units;
  a.cstride = p.cstride;
  a.ws_keys = p.keys_bytes ? (uint64_t*)scratch : nullptr;
  a.ws_part = p.part_bytes ? (float*)((char*)scratch + keys_at) : nullptr;
  a.lists = lists; a.lengths = lengths; a.status = status;
  a.slots = sm;
  const dim3 g3((unsigned)grid);
  hipStream_t s = (hipStream_t)stream;
  const bool bf16 = score_mode == LSA_SCORE_BF16;
  if (dtype == LSA_BF16) decode::launch_bf16(a, p.rep, bf16, D, gq, g3, p.shmem, s);
  else if (dtype == LSA_F16) decode::launch_f16(a, p.rep, bf16, D, gq, g3, p.shmem, s);
  else decode::launch_f32(a, p.rep, bf16, D, gq, g3, p.shmem, s);
  LSA_LAUNCHED(who);
  return LSA_OK;
}

}  // namespace

extern "C" int lsa_decode_flat(const void* q, const void* k, const void* v, int dtype, int64_t R, int64_t Tk,
                               int32_t Hq, int32_t Hkv, int32_t D, int64_t kv_batch_stride, int64_t kv_token_stride,
                               int64_t kv_head_stride, const void* centroids, const int32_t* members,
                               const int32_t* ends, int32_t table_flags, int32_t rows, int32_t cap, int64_t row_tables,
                               int64_t group_tables, int score_mode, const int32_t* positions,
                               const lsa_slot_map* slots, int32_t cluster_block_size, int32_t block_buckets,
                               int32_t top_p, int32_t window, int32_t sink, int32_t top_k, float scale,
                               int32_t select_splits, int32_t readers, int32_t* counters, int64_t n_counters,
                               void* scratch, size_t scratch_bytes, int32_t* lists, int32_t* lengths, void* out,
                               int32_t* status, void* stream) {
  return decode_launch("lsa_decode_flat", q, k, v, dtype, R, Tk, Hq, Hkv, D, kv_batch_stride, kv_token_stride,
                       kv_head_stride, centroids, members, ends, table_flags, rows, cap, row_tables, group_tables,
                       score_mode, positions, slots, cluster_block_size, block_buckets, top_p, window, sink, top_k,
                       scale,
                       select_splits, readers, counters, n_counters, scratch, scratch_bytes, lists, lengths, out,
                       status, stream, nullptr);
}

extern "C" int lsa_decode_tree(const void* q, const void* k, const void* v, int dtype, int64_t R, int64_t Tk,
                               int32_t Hq, int32_t Hkv, int32_t D, int64_t kv_batch_stride, int64_t kv_token_stride,
                               int64_t kv_head_stride, const void* node_centroids, const int32_t* children,
                               int32_t n_nodes, int32_t node_size, int32_t node_block, int32_t beam_width,
                               const void* centroids, const int32_t* members, const int32_t* ends,
                               int32_t table_flags, int32_t rows, int32_t cap, int64_t row_tables,
                               int64_t group_tables, int score_mode, const int32_t* positions,
                               const lsa_slot_map* slots, int32_t cluster_block_size, int32_t block_buckets,
                               int32_t top_p, int32_t window, int32_t sink, int32_t top_k, float scale,
                               int32_t readers, int32_t* counters, int64_t n_counters, void* scratch,
                               size_t scratch_bytes, int32_t* lists, int32_t* lengths, void* out, int32_t* status,
                               void* stream) {
  const TreeSpec tree{node_centroids, children, n_nodes, node_size, node_block, beam_width};
  return decode_launch("lsa_decode_tree", q, k, v, dtype, R, Tk, Hq, Hkv, D, kv_batch_stride, kv_token_stride,
                       kv_head_stride, centroids, members, ends, table_flags, rows, cap, row_tables, group_tables,
                       score_mode, positions, slots, cluster_block_size, block_buckets, top_p, window, sink, top_k,
                       scale, 1,
                       readers, counters, n_counters, scratch, scratch_bytes, lists, lengths, out, status, stream,
                       &tree);
}
