// MFMA tile kernel for the chunked prefill read (bf16, head dim 128).
#include "lsa_abi_common.h"
