// Host-only helpers of the C ABI (no device code).
#include <hip/hip_runtime_api.h>

#include "../../include/qf_attn.h"

extern "C" const char* qf_error_string(int code) {
  if (code == QF_OK) return "success";
  if (code == QF_ERR_INVALID_ARG)
    return "invalid argument (null pointer, bad size, misaligned pointer or stride)";
  if (code == QF_ERR_UNSUPPORTED) return "unsupported shape (requires head_dim 64 and 1 <= G <= 16)";
  if (code == QF_ERR_SCRATCH_LIMIT)
    return "problem too large for the no-allocation scratch "
           "(B*KVH*splits*G*(D+2)*4 bytes > QF_NOALLOC_PARTIAL_BYTES)";
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "unknown error";
}

// major * 100 + minor.  301: qf_decode_split_capacity added.  300:
// qf_attn_merge_o_proj and qf_rms_lm_head take a weight-layout argument, and
// the single-launch decode ticket is one counter per (b, kv head).  200: the
// prefill workspace entry points were removed.
extern "C" int qf_abi_version(void) { return 301; }
