// Fused decode kernels with bf16_t queries and K/V rows.
#include "decode_dev.h"

namespace lsa {
namespace decode {

void launch_bf16(const DecodeArgs& a, bool rep, bool bf16_table, int D, int gq, dim3 grid, size_t shmem,
                 hipStream_t s) {
  launch_type<bf16_t>(a, rep, bf16_table, D, gq, grid, shmem, s);
}

}  // namespace decode
}  // namespace lsa
