// Instantiations of the dense OUTPUT pass for fp32 V (fp32 / bf16 outputs).
#include "dense_kernel.h"

namespace mogt {
template int dense_launch_pass<float, float, CM_OUTPUT>(const ChunkParams&, int64_t, hipStream_t);
template int dense_launch_pass<float, bf16_t, CM_OUTPUT>(const ChunkParams&, int64_t, hipStream_t);
}  // namespace mogt
