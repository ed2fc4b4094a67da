// Instantiations of the dense chunk passes that produce and consume chunk
// summaries: SUMMARY (level-0 inputs fp32 / bf16) and EXCL (upper levels, fp32).
#include "dense_kernel.h"

namespace mogt {
template int dense_launch_pass<float, float, CM_SUMMARY>(const ChunkParams&, int64_t, hipStream_t);
template int dense_launch_pass<bf16_t, float, CM_SUMMARY>(const ChunkParams&, int64_t, hipStream_t);
template int dense_launch_pass<float, float, CM_EXCL>(const ChunkParams&, int64_t, hipStream_t);
}  // namespace mogt
