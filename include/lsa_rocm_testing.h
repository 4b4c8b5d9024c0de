/* Test hooks of liblsa_rocm.so: not part of the drop-in interface (include/lsa_rocm.h).
 * The library exports them so that tests can drive failure paths from the host. */
#ifndef LSA_ROCM_TESTING_H
#define LSA_ROCM_TESTING_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Thread-local, this thread's later fused-decode calls (lsa_decode_flat, lsa_decode_tree,
 * lsa_decode_shared, lsa_decode_tree_shared): skip_publish != 0 makes the select
 * workgroups skip publishing the record or their keys, and spin_limit > 0 replaces the
 * readers' poll limit, so a test can make the bounded wait give up with every workgroup
 * still exiting normally. lsa_debug_decode(0, 0) restores the defaults. No counterpart in
 * the reference (its decode has no cross-workgroup wait). */
void lsa_debug_decode(int32_t skip_publish, int32_t spin_limit);

#ifdef __cplusplus
}
#endif

#endif /* LSA_ROCM_TESTING_H */
