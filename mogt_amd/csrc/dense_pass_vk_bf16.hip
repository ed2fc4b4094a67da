// Instantiations of the level-0 dense OUTPUT pass with V_t = v_t k_t^T formed in
// registers, bf16 output.
#include "dense_kernel.h"

namespace mogt {
template int dense_launch_pass<float, bf16_t, CM_OUTPUT, true>(const ChunkParams&, int64_t, hipStream_t);
template int dense_launch_pass<bf16_t, bf16_t, CM_OUTPUT, true>(const ChunkParams&, int64_t, hipStream_t);
}  // namespace mogt
