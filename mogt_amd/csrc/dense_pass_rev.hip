// Instantiations of the reverse-time level-0 dense passes (the backward's
// G_t = X_t + U_{t+1}^T G_{t+1}): SUMMARY and OUTPUT, fp32.
#include "dense_kernel.h"

namespace mogt {
template int dense_launch_pass<float, float, CM_SUMMARY, false, true>(const ChunkParams&, int64_t, hipStream_t);
template int dense_launch_pass<float, float, CM_OUTPUT, false, true>(const ChunkParams&, int64_t, hipStream_t);
}  // namespace mogt
