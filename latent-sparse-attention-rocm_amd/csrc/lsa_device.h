// Device building blocks shared by the select and read kernels (gfx950, wave64).
//
// Packed selection keys follow the reference layout (select_fused.py:71-77):
//   key = (ordered_bits(score) << 32) | (0x7FFFFFFF - column),   EMPTY = INT64_MIN
// Inside a workgroup keys are handled as u = key ^ 0x8000000000000000, an unsigned
// value with the same order, so EMPTY is u == 0 and "best first" is "largest u first".
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define LSA_BLOCK 256
#define LSA_WAVE 64
#define LSA_WAVES (LSA_BLOCK / LSA_WAVE)

namespace lsa {

constexpr int64_t kEmpty = (int64_t)0x8000000000000000ull;
constexpr uint64_t kSignBit = 0x8000000000000000ull;
// Partial sums per canonical dot product (16 lanes, tree (p,p+8),(p,p+4),(p,p+2),(p,p+1)).
constexpr int kScorePartials = 16;

struct bf16_t { uint16_t bits; };

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// fp32 -> bf16, round to nearest even; NaN -> 0x7FC0 (torch's conversion).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return 0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

template <typename T> struct elem;
template <> struct elem<float> {
  static __device__ __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void store(float* p, int64_t i, float x) { p[i] = x; }
};
template <> struct elem<bf16_t> {
  static __device__ __forceinline__ float load(const bf16_t* p, int64_t i) { return bf16_to_f32(p[i].bits); }
  static __device__ __forceinline__ void store(bf16_t* p, int64_t i, float x) { p[i].bits = f32_to_bf16(x); }
};
template <> struct elem<_Float16> {
  static __device__ __forceinline__ float load(const _Float16* p, int64_t i) { return (float)p[i]; }
  static __device__ __forceinline__ void store(_Float16* p, int64_t i, float x) { p[i] = (_Float16)x; }
};

// ---------------------------------------------------------------- packed keys

__device__ __forceinline__ int32_t ordered_bits(float s) {
  int32_t b = __float_as_int(s);
  return b ^ ((b >> 31) & 0x7FFFFFFF);
}

__device__ __forceinline__ int64_t pack_key(float s, int32_t column) {
  uint64_t hi = (uint64_t)(uint32_t)ordered_bits(s) << 32;
  return (int64_t)(hi | (uint64_t)(uint32_t)(0x7FFFFFFF - column));
}

__device__ __forceinline__ uint64_t key_to_u(int64_t key) { return (uint64_t)key ^ kSignBit; }
__device__ __forceinline__ int64_t u_to_key(uint64_t u) { return (int64_t)(u ^ kSignBit); }

// Column of a key; -1 for EMPTY (upstream key_bucket / unpack_ids).
__device__ __forceinline__ int32_t key_column(int64_t key) {
  if (key == kEmpty) return -1;
  return 0x7FFFFFFF - (int32_t)(uint32_t)((uint64_t)key & 0xFFFFFFFFull);
}

// ---------------------------------------------------------------- wave / block scans

// DPP lane exchange inside a row of 16: dpp_ctrl quad_perm / row mirrors.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// v_permlane16_swap / v_permlane32_swap of a and b (gfx950): the odd 16-lane rows of a
// trade places with the even rows of b (16), or a's upper 32 lanes with b's lower 32 (32).
// Written as instructions: this compiler's builtins mis-model the swap's second result when
// both results feed one expression (it reuses the first). s_nop 1: the wait states a swap
// needs after a VALU write of its operands.
__device__ __forceinline__ void row_swap16(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void row_swap32(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}

// The partner value of lane ^ x for x in {16, 32} (v_permlane16/32_swap of two copies),
// else a bpermute shuffle. The builtins serve here: each result is used alone.
__device__ __forceinline__ float lane_xor(float v, int x) {
  const int iv = __builtin_bit_cast(int, v);
  const int row = (threadIdx.x & (LSA_WAVE - 1)) >> 4;
  if (x == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(iv, iv, false, false);  // [v0, v0, v2, v2], [v1, v1, v3, v3]
    return __builtin_bit_cast(float, (row & 1) ? r[0] : r[1]);
  }
  if (x == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(iv, iv, false, false);  // [v0, v1, v0, v1], [v2, v3, v2, v3]
    return __builtin_bit_cast(float, (row & 2) ? r[0] : r[1]);
  }
  return __shfl_xor(v, x, LSA_WAVE);
}

// Cross-lane moves by DPP (the data-parallel primitives of the VALU, no LDS round trip):
// the lane's value from the lane named by `ctrl`, or `ident` where the control names no
// source lane or the lane's row is outside `row_mask`.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int dpp_or(int ident, int x) {
  return __builtin_amdgcn_update_dpp(ident, x, CTRL, ROW_MASK, 0xF, false);
}
constexpr int kDppXor1 = 0xB1;      // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;      // quad_perm [2, 3, 0, 1]
constexpr int kDppRowShr1 = 0x111;  // row_shr:n = 0x110 + n
constexpr int kDppRowShr2 = 0x112;
constexpr int kDppRowShr4 = 0x114;
constexpr int kDppRowShr8 = 0x118;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;
constexpr int kDppBcast15 = 0x142;  // lane 15 of each row to the next row
constexpr int kDppBcast31 = 0x143;  // lane 31 to rows 2 and 3
constexpr int kDppWaveShr1 = 0x138; // the whole wave shifted up one lane (lane 0 has no source)

// Wave-wide reduction of an associative, commutative op with identity `ident` (int bits):
// pairs, quads, 8-lane halves and rows by DPP, then rows 1 and 3 take their lower
// neighbour's total and rows 2 and 3 take lane 31's; lane 63 ends with the whole wave's,
// which every lane reads.
template <typename Op>
__device__ __forceinline__ int wave_reduce_bits(int x, int ident, Op op) {
  x = op(x, dpp_or<kDppXor1>(ident, x));
  x = op(x, dpp_or<kDppXor2>(ident, x));
  x = op(x, dpp_or<kDppHalfMirror>(ident, x));
  x = op(x, dpp_or<kDppMirror>(ident, x));
  x = op(x, dpp_or<kDppBcast15, 0xA>(ident, x));
  x = op(x, dpp_or<kDppBcast31, 0xC>(ident, x));
  return __builtin_amdgcn_readlane(x, LSA_WAVE - 1);
}
__device__ __forceinline__ int wave_sum(int x) {
  return wave_reduce_bits(x, 0, [](int a, int b) { return a + b; });
}
__device__ __forceinline__ int wave_or(int x) {
  return wave_reduce_bits(x, 0, [](int a, int b) { return a | b; });
}
__device__ __forceinline__ float wave_sum(float x) {  // a fixed order: the same bits every run
  return __int_as_float(wave_reduce_bits(__float_as_int(x), 0, [](int a, int b) {
    return __float_as_int(__int_as_float(a) + __int_as_float(b));
  }));
}
__device__ __forceinline__ float wave_max(float x) {
  return __int_as_float(wave_reduce_bits(__float_as_int(x), __float_as_int(-INFINITY), [](int a, int b) {
    return __float_as_int(fmaxf(__int_as_float(a), __int_as_float(b)));
  }));
}
__device__ __forceinline__ float wave_min(float x) {
  return __int_as_float(wave_reduce_bits(__float_as_int(x), __float_as_int(INFINITY), [](int a, int b) {
    return __float_as_int(fminf(__int_as_float(a), __int_as_float(b)));
  }));
}

// Inclusive prefix sum over the wave's lanes: Hillis-Steele within each 16-lane row by DPP
// row shifts (a lane with no source adds 0), then rows 1 and 3 add their lower neighbour's
// total and rows 2 and 3 add lane 31's.
__device__ __forceinline__ int wave_inclusive_sum(int x) {
  x += dpp_or<kDppRowShr1>(0, x);
  x += dpp_or<kDppRowShr2>(0, x);
  x += dpp_or<kDppRowShr4>(0, x);
  x += dpp_or<kDppRowShr8>(0, x);
  x += dpp_or<kDppBcast15, 0xA>(0, x);
  x += dpp_or<kDppBcast31, 0xC>(0, x);
  return x;
}

// Exclusive prefix sum over the 256 threads; *total receives the block sum.
// `scratch` holds LSA_WAVES ints. Contains barriers: every thread must call it.
__device__ __forceinline__ int block_exclusive_sum(int x, int* scratch, int* total) {
  const int lane = threadIdx.x & (LSA_WAVE - 1);
  const int wave = threadIdx.x / LSA_WAVE;
  int inc = wave_inclusive_sum(x);
  if (lane == LSA_WAVE - 1) scratch[wave] = inc;
  __syncthreads();
  int before = 0, sum = 0;
#pragma unroll
  for (int w = 0; w < LSA_WAVES; ++w) {
    int v = scratch[w];
    before += (w < wave) ? v : 0;
    sum += v;
  }
  __syncthreads();
  *total = sum;
  return before + inc - x;
}

// ---------------------------------------------------------------- radix select

// State of a top-k radix select, kept in LDS by the caller.
struct RadixState {
  uint64_t prefix;     // selected high digits
  uint64_t mask;       // which bits of prefix are fixed
  int need;            // how many keys equal to (prefix-range) are still needed
  int done;            // 1: every key >= prefix is selected (early exit)
  int hist[256];
  int slot;            // collection cursor
};

// Finds the k-th largest of the n values produced by get(i) (u-ordered keys).
// On return (after a barrier) the selected set is either
//   done == 1: every value v >= prefix (its low digits are zero), exactly k of them;
//   done == 0: every value > prefix plus `need` copies of prefix (ties).
// 1 <= k <= n. Every thread of the block must call it.
template <typename Get>
__device__ __forceinline__ void radix_select(Get get, int n, int k, RadixState* st) {
  const int tid = threadIdx.x;
  if (tid == 0) { st->prefix = 0; st->mask = 0; st->need = k; st->done = 0; }
  for (int pass = 0; pass < 8; ++pass) {
    const int shift = 56 - 8 * pass;
    st->hist[tid] = 0;  // LSA_BLOCK == 256 bins
    __syncthreads();
    const uint64_t prefix = st->prefix, mask = st->mask;
    for (int i = tid; i < n; i += LSA_BLOCK) {
      uint64_t v = get(i);
      if ((v & mask) == prefix) atomicAdd(&st->hist[(v >> shift) & 255], 1);
    }
    __syncthreads();
    if (tid < LSA_WAVE) {
      // lane l owns bins 255-4l .. 252-4l (descending); suffix counts from the top bin
      int c0 = st->hist[255 - 4 * tid], c1 = st->hist[254 - 4 * tid];
      int c2 = st->hist[253 - 4 * tid], c3 = st->hist[252 - 4 * tid];
      int mine = c0 + c1 + c2 + c3;
      int inc = wave_inclusive_sum(mine);
      int above = inc - mine;  // count in bins above this lane's group
      const int need = st->need;
      if (above < need && need <= inc) {
        int d = 255 - 4 * tid, cnt = c0;
        if (above + c0 < need) { above += c0; d -= 1; cnt = c1;
          if (above + c1 < need) { above += c1; d -= 1; cnt = c2;
            if (above + c2 < need) { above += c2; d -= 1; cnt = c3; } } }
        const int rest = need - above;
        st->prefix = prefix | ((uint64_t)d << shift);
        st->mask = mask | (0xFFull << shift);
        st->need = rest;
        st->done = (cnt == rest) ? 1 : 0;
      }
    }
    __syncthreads();
    if (st->done) break;
  }
}

// Appends the selected values (see radix_select) to out[0..k) in arbitrary order.
template <typename Get>
__device__ __forceinline__ void radix_collect(Get get, int n, int k, RadixState* st, uint64_t* out) {
  const int tid = threadIdx.x;
  if (tid == 0) st->slot = 0;
  __syncthreads();
  const uint64_t prefix = st->prefix;
  const int done = st->done;
  for (int i = tid; i < n; i += LSA_BLOCK) {
    uint64_t v = get(i);
    bool take = done ? (v >= prefix) : (v > prefix);
    if (take) out[atomicAdd(&st->slot, 1)] = v;
  }
  __syncthreads();
  if (!done) {
    const int base = st->slot;  // == k - need
    for (int i = base + tid; i < k; i += LSA_BLOCK) out[i] = prefix;
  }
  __syncthreads();
}

// Sorts a[0..n) descending in LDS; n is a power of two. Every thread must call it.
__device__ __forceinline__ void bitonic_sort_desc(uint64_t* a, int n) {
  const int tid = threadIdx.x;
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < n / 2; i += LSA_BLOCK) {
        int lo = 2 * i - (i & (stride - 1));
        int hi = lo + stride;
        bool desc = ((lo & size) == 0);
        uint64_t x = a[lo], y = a[hi];
        if ((x < y) == desc) { a[lo] = y; a[hi] = x; }
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------- paged caches

// A paged cache's slot table, by value in kernel arguments (table == nullptr: ids are
// cache rows). Row r of the query rows maps logical position p to table[rows[r] * stride + p].
struct SlotMap {
  const int32_t* table;
  const int32_t* rows;
  int64_t stride;
  int32_t width;   // positions a table row maps; ids at or past it map to -1
  int32_t n_rows;  // table rows; a row index outside [0, n_rows) maps every id to -1
};

// One query row's view of the slot table: map(id) is the physical cache row of logical
// position id (-1 stays -1; ids outside [0, width) map to -1); the identity without a table.
struct SlotRow {
  const int32_t* row;  // nullptr: identity
  int32_t width;
  __device__ __forceinline__ int32_t operator()(int32_t id) const {
    if (row == nullptr || id < 0) return id;
    return id < width ? row[id] : -1;
  }
};

// The slot row of query row r (one load of rows[r], issued where called).
__device__ __forceinline__ SlotRow slot_row_of(const SlotMap& m, int64_t r) {
  SlotRow s{nullptr, 0};
  if (m.table != nullptr) {
    const int32_t k = m.rows[r];
    const bool ok = k >= 0 && k < m.n_rows;
    s.row = m.table + (ok ? (int64_t)k : 0) * m.stride;
    s.width = ok ? m.width : 0;  // a bad row index maps everything to -1
  }
  return s;
}

// ---------------------------------------------------------------- cross-workgroup exchange

// Values handed between workgroups that may sit on different XCDs (whose L2s are not
// coherent with each other) go through device-scope accesses (the sc1 cache policy):
// relaxed agent-scope atomic loads and stores, coherent across the XCDs. Publishing then
// needs only the stores' completion (s_waitcnt) before an arrival counter, never a
// device-scope release fence (a whole-L2 writeback on gfx950). System-scope (volatile,
// sc0 sc1) accesses would also be coherent but move data ~3x slower per workgroup.
__device__ __forceinline__ void coherent_store_u64(uint64_t* p, uint64_t x) {
  __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t coherent_load_u64(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coherent_store_i32(int32_t* p, int32_t x) {
  __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t coherent_load_i32(const int32_t* p) {
  return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coherent_store(float* p, float x) {
  __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float coherent_load(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16-byte device-scope loads from a workgroup-uniform base: a buffer resource over `base`
// and per-lane byte offsets (buffer_load_dwordx4 ... sc1).
struct CoherentRows {
  __amdgpu_buffer_rsrc_t rsrc;
  __device__ __forceinline__ explicit CoherentRows(const float* base)
      : rsrc(__builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, 0x7FFFFFFF, 0x00020000)) {}
  __device__ __forceinline__ float4 load4(int byte_offset) const {
    typedef float f4v __attribute__((ext_vector_type(4)));
    const f4v v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, byte_offset, 0, 16 /* sc1 */);
    return make_float4(v[0], v[1], v[2], v[3]);
  }
};

// Every thread's coherent stores complete, then one arrival on `counter`; returns (to
// every thread) whether this workgroup arrived last of `expected`. The last one resets the
// counter to zero for the next launch. Contains barriers: every thread calls it.
__device__ __forceinline__ bool arrive_last(int* counter, int expected, int* flag) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int before = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = before == expected - 1;
    if (before == expected - 1) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  const bool last = *flag != 0;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return last;
}

// ---------------------------------------------------------------- wave top-k

// One wave selects the K (<= 64) largest of keys[0..n) (u-ordered, n <= 64 * KPL) and
// writes them sorted descending to out[0..kp), u == 0 past K. Nonzero keys are distinct
// (a packed key carries its column); only u == 0 (EMPTY) repeats. The K-th largest value
// T is found bit by bit, high word first, by wave-wide counts (ballot + popcount, no
// barriers); the keys above T and then copies of T are compacted into tmp[0..K) and
// ranked into place. Called by the 64 threads of one wave.
template <int KPL>
__device__ __forceinline__ void wave_topk_sorted(const uint64_t* keys, int n, int K, int kp, uint64_t* out,
                                                 uint64_t* tmp) {
  const int lane = threadIdx.x & (LSA_WAVE - 1);
  uint32_t vh[KPL], vl[KPL];
#pragma unroll
  for (int j = 0; j < KPL; ++j) {
    const int idx = lane + LSA_WAVE * j;
    const uint64_t v = idx < n ? keys[idx] : 0;
    vh[j] = (uint32_t)(v >> 32);
    vl[j] = (uint32_t)v;
  }
  // high word of T: the largest h with #(high >= h) >= K
  uint32_t hi = 0;
  for (int b = 31; b >= 0; --b) {
    const uint32_t cand = hi | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < KPL; ++j) cnt += __popcll(__ballot(vh[j] >= cand));
    if (cnt >= K) hi = cand;
  }
  int above = 0, at_hi = 0;
#pragma unroll
  for (int j = 0; j < KPL; ++j) {
    above += __popcll(__ballot(vh[j] > hi));
    at_hi += __popcll(__ballot(vh[j] == hi));
  }
  uint32_t lo = 0;
  if (above + at_hi > K) {  // the K-th key shares its high word with keys below it
    const int need = K - above;
    for (int b = 31; b >= 0; --b) {
      const uint32_t cand = lo | (1u << b);
      int cnt = 0;
#pragma unroll
      for (int j = 0; j < KPL; ++j) cnt += __popcll(__ballot(vh[j] == hi && vl[j] >= cand));
      if (cnt >= need) lo = cand;
    }
  }
  const uint64_t T = ((uint64_t)hi << 32) | lo;
  // compact the keys above T, then fill with T (repeats only when T is EMPTY)
  int base = 0;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (LSA_WAVE - lane));
#pragma unroll
  for (int j = 0; j < KPL; ++j) {
    const uint64_t v = ((uint64_t)vh[j] << 32) | vl[j];
    const bool take = v > T;
    const uint64_t m = __ballot(take);
    if (take) tmp[base + __popcll(m & below)] = v;
    base += __popcll(m);
  }
  for (int m = base + lane; m < K; m += LSA_WAVE) tmp[m] = T;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  if (lane < K) {
    const uint64_t x = tmp[lane];
    int rank = 0;
    for (int m = 0; m < K; ++m) {
      const uint64_t y = tmp[m];
      rank += (y > x || (y == x && m < lane)) ? 1 : 0;
    }
    out[rank] = x;
  }
  for (int m = K + lane; m < kp; m += LSA_WAVE) out[m] = 0;
}

// ---------------------------------------------------------------- canonical score

// The value of lane ^ X (X in {1, 2, 4, 8}: within a 16-lane row) by DPP: quad
// permutations for 1 and 2; for 4 and 8, row shifts up and down on the 4-lane banks that
// take their partner from above or below.
template <int X>
__device__ __forceinline__ int xor_dpp_bits(int x) {
  if constexpr (X == 1) return __builtin_amdgcn_update_dpp(x, x, kDppXor1, 0xF, 0xF, false);
  if constexpr (X == 2) return __builtin_amdgcn_update_dpp(x, x, kDppXor2, 0xF, 0xF, false);
  if constexpr (X == 4) {
    const int t = __builtin_amdgcn_update_dpp(x, x, 0x104, 0xF, 0x5, false);  // row_shl:4, banks 0, 2
    return __builtin_amdgcn_update_dpp(t, x, 0x114, 0xF, 0xA, false);         // row_shr:4, banks 1, 3
  }
  const int t = __builtin_amdgcn_update_dpp(x, x, 0x108, 0xF, 0x3, false);    // row_shl:8, banks 0, 1
  return __builtin_amdgcn_update_dpp(t, x, 0x118, 0xF, 0xC, false);           // row_shr:8, banks 2, 3
}
template <int X>
__device__ __forceinline__ double xor_dpp(double v) {
  const uint64_t b = __double_as_longlong(v);
  const int lo = xor_dpp_bits<X>((int)(uint32_t)b), hi = xor_dpp_bits<X>((int)(uint32_t)(b >> 32));
  return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}

// One canonical dot product shared by 16 lanes: lane p (0..15 within its group) has
// already summed dims [p*span, (p+1)*span) in order into `partial` (fp64).
// Returns the fp32 score in every lane of the 16-lane group.
__device__ __forceinline__ float score_tree16(double partial) {
  partial += xor_dpp<8>(partial);
  partial += xor_dpp<4>(partial);
  partial += xor_dpp<2>(partial);
  partial += xor_dpp<1>(partial);
  return (float)partial;
}

// Scores one centroid row against a query slice held by the lane: q[j] are the lane's
// span query values (already rounded to the scoring type), c points at the row.
template <typename C>
__device__ __forceinline__ double partial_dot(const float* q, const C* c, int span, int p) {
  double acc = 0.0;
  const C* base = c + (int64_t)p * span;
#pragma unroll 4
  for (int j = 0; j < span; ++j) acc = fma((double)q[j], (double)elem<C>::load(base, j), acc);
  return acc;
}

}  // namespace lsa
