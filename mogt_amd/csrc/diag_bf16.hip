// Instantiations of the single-pass diagonal scan for bf16 inputs (see diag_kernel.h).
#include "diag_kernel.h"

namespace mogt {

int diag_run_bf16in(const DiagParams& prm, const DiagTile& t, int out_dtype, bool prefix,
                    hipStream_t st) {
#define MOGT_CASE(V_, F_, S_, W_)                                                                        \
    if (t.vec == V_ && t.lanes == F_ && t.steps == S_ && t.waves == W_) {                                             \
        if (out_dtype == MOGT_F32)                                                                   \
            return prefix ? diag_launch<MODE_DIAG, bf16_t, float, float, V_, F_, S_, W_, true>(prm, st)   \
                          : diag_launch<MODE_DIAG, bf16_t, float, float, V_, F_, S_, W_, false>(prm, st); \
        return prefix ? diag_launch<MODE_DIAG, bf16_t, float, bf16_t, V_, F_, S_, W_, true>(prm, st)      \
                      : diag_launch<MODE_DIAG, bf16_t, float, bf16_t, V_, F_, S_, W_, false>(prm, st);    \
    }
    MOGT_DIAG_BF16_TILES(MOGT_CASE)
#undef MOGT_CASE
    return set_error(MOGT_E_INVALID, "diag scan: tile (vec=%d, lanes=%d, steps=%d, waves=%d) not compiled for bf16 input",
                     t.vec, t.lanes, t.steps, t.waves);
}

}  // namespace mogt
