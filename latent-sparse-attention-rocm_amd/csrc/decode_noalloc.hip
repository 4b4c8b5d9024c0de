// The fused decode step for callers that cannot allocate (code under HIP graph capture,
// tight serving loops): lsa_decode_flat with its arrival counters and scratch taken from a
// file-scope device array instead of caller buffers. No hipMalloc, hipFree or allocating
// library call anywhere on this path.
//
// Each GPU holds its own copy of `scratch` for the life of the process. Its address on a
// device comes from hipGetSymbolAddress, called once per device with that device current;
// the host never passes the array's name to a kernel or a copy (in host code the name is a
// host-side stand-in, not a device address). The first call on a device clears the
// counters region with a fill kernel on the caller's stream; every decode launch leaves
// the counters zero again, so later calls need no clearing. Calls share the array: two
// calls that overlap on one GPU (different streams, or threads) race and must not.
#include <mutex>

#include "lsa_abi_common.h"

namespace {

constexpr size_t kScratchBytes = 16u << 20;      // the whole array: 16 MiB per GPU
constexpr int64_t kCounterWords = 256 * 1024;    // int32 counters at the start (1 MiB)
constexpr size_t kCounterBytes = (size_t)kCounterWords * sizeof(int32_t);
constexpr int kMaxDevices = 64;

static __device__ __align__(256) char scratch[kScratchBytes];

std::mutex g_lock;
char* g_base[kMaxDevices];  // per device: the array's device address, set once

__global__ void zero_words(int32_t* p, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0;
}

// The array's address on the current device; the first call on a device resolves it and
// clears the counters on `stream`.
int scratch_base(hipStream_t stream, char** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  LSA_REQUIRE(err == hipSuccess, LSA_ERR_LAUNCH, "lsa_decode_flat_noalloc: hipGetDevice: %s", hipGetErrorString(err));
  LSA_REQUIRE(dev >= 0 && dev < kMaxDevices, LSA_ERR_LAUNCH, "lsa_decode_flat_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> guard(g_lock);
  if (g_base[dev] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    LSA_REQUIRE(err == hipSuccess && ptr != nullptr, LSA_ERR_LAUNCH,
                "lsa_decode_flat_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(err));
    zero_words<<<64, 256, 0, stream>>>((int32_t*)ptr, kCounterWords);
    LSA_LAUNCHED("lsa_decode_flat_noalloc (counter clear)");
    g_base[dev] = (char*)ptr;
  }
  *out = g_base[dev];
  return LSA_OK;
}

}  // namespace

extern "C" int lsa_decode_flat_noalloc(const void* q, const void* k, const void* v, int dtype, int64_t R, int64_t Tk,
                                       int32_t Hq, int32_t Hkv, int32_t D, int64_t kv_batch_stride,
                                       int64_t kv_token_stride, int64_t kv_head_stride, const void* centroids,
                                       const int32_t* members, const int32_t* ends, int32_t table_flags, int32_t rows,
                                       int32_t cap, int64_t row_tables, int64_t group_tables, int score_mode,
                                       const int32_t* positions, int32_t cluster_block_size, int32_t block_buckets,
                                       int32_t top_p, int32_t window, int32_t sink, int32_t top_k, float scale,
                                       int32_t select_splits, int32_t readers, int32_t reset_counters,
                                       int32_t* lists, int32_t* lengths, void* out, int32_t* status, void* stream) {
  LSA_REQUIRE(Hkv >= 1 && Hq >= Hkv && R >= 0, LSA_ERR_SHAPE, "lsa_decode_flat_noalloc: bad sizes");
  if (R == 0) return LSA_OK;
  const int64_t n_counters = lsa_decode_flat_counters(R, Hkv, rows, top_p);
  LSA_REQUIRE(n_counters > 0, LSA_ERR_SHAPE, "lsa_decode_flat_noalloc: unsupported table or pick count");
  LSA_REQUIRE(n_counters <= kCounterWords, LSA_ERR_WORKSPACE,
              "lsa_decode_flat_noalloc: %lld counter words exceed the %lld this entry point holds; use "
              "lsa_decode_flat with a caller workspace",
              (long long)n_counters, (long long)kCounterWords);
  const size_t need = lsa_decode_flat_scratch_bytes(dtype, R, Hq, Hkv, D, rows, top_p, window, sink, select_splits,
                                                    readers);
  LSA_REQUIRE(need <= kScratchBytes - kCounterBytes, LSA_ERR_WORKSPACE,
              "lsa_decode_flat_noalloc: %zu scratch bytes exceed the %zu this entry point holds; use "
              "lsa_decode_flat with a caller workspace",
              need, kScratchBytes - kCounterBytes);
  hipStream_t s = (hipStream_t)stream;
  char* base = nullptr;
  LSA_TRY(scratch_base(s, &base));
  if (reset_counters) {
    // after a launch gave up waiting (status set): a late select split of that launch may
    // have left published keys or record words anywhere its own (perhaps larger) shape
    // reached, so the whole counters region is cleared, not only this call's words
    zero_words<<<64, 256, 0, s>>>((int32_t*)base, kCounterWords);
    LSA_LAUNCHED("lsa_decode_flat_noalloc (counter reset)");
  }
  return lsa_decode_flat(q, k, v, dtype, R, Tk, Hq, Hkv, D, kv_batch_stride, kv_token_stride, kv_head_stride,
                         centroids, members, ends, table_flags, rows, cap, row_tables, group_tables, score_mode,
                         positions, nullptr, cluster_block_size, block_buckets, top_p, window, sink, top_k, scale,
                         select_splits, readers, (int32_t*)base, n_counters, need ? base + kCounterBytes : nullptr,
                         need, lists, lengths, out, status, stream);
}
