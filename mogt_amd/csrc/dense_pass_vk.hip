// Instantiations of the level-0 dense passes whose V_t = v_t k_t^T is formed in
// registers from the vectors v and k (SUMMARY; OUTPUT with fp32 output).
#include "dense_kernel.h"

namespace mogt {
template int dense_launch_pass<float, float, CM_SUMMARY, true>(const ChunkParams&, int64_t, hipStream_t);
template int dense_launch_pass<bf16_t, float, CM_SUMMARY, true>(const ChunkParams&, int64_t, hipStream_t);
template int dense_launch_pass<float, float, CM_OUTPUT, true>(const ChunkParams&, int64_t, hipStream_t);
template int dense_launch_pass<bf16_t, float, CM_OUTPUT, true>(const ChunkParams&, int64_t, hipStream_t);
}  // namespace mogt
