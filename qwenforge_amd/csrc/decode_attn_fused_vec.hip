// The decode split kernel's single-launch-merge instances with a 16-byte bias
// over a contiguous cache (decode_split_kernel<NW, kBiasVec, kFused, false>),
// compiled on their own so that qwenforge_amd/build.py can give this unit
// LLVM's max-ILP machine scheduler (-mllvm -amdgpu-sched-strategy=max-ilp)
// while decode_attn.hip keeps the default: the flag applies to a whole unit
// and helps these instances only.  decode_attn.hip launches them through
// qf::launch_fused_vec.
#define QF_DECODE_FUSED_VEC_UNIT
#include "decode_attn.hip"
