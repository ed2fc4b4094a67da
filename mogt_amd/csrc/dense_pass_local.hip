// Instantiations of the dense LOCAL pass (block-local scan of any block size).
#include "dense_kernel.h"

namespace mogt {
template int dense_launch_pass<float, float, CM_LOCAL>(const ChunkParams&, int64_t, hipStream_t);
template int dense_launch_pass<bf16_t, float, CM_LOCAL>(const ChunkParams&, int64_t, hipStream_t);
}  // namespace mogt
