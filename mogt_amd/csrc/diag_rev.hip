// Instantiations of the reverse-time diagonal scan (the backward recurrence
// G_t = dH_t + a_{t+1} G_{t+1}, see MODE_DIAG_REV in diag_kernel.h): fp32 in,
// fp32 out, the tiles of the fp32 default lists.
#include "diag_kernel.h"

namespace mogt {

#define MOGT_DIAG_REV_TILES(X) X(2, 32, 32, 8) X(2, 32, 16, 8) X(2, 32, 8, 16) X(1, 64, 32, 16) X(1, 64, 16, 16) X(1, 64, 8, 16)

int diag_run_rev(const DiagParams& prm, const DiagTile& t, hipStream_t st) {
#define MOGT_CASE(V_, F_, S_, W_)                                                         \
    if (t.vec == V_ && t.lanes == F_ && t.steps == S_ && t.waves == W_)                   \
        return diag_launch<MODE_DIAG_REV, float, float, float, V_, F_, S_, W_, false>(prm, st);
    MOGT_DIAG_REV_TILES(MOGT_CASE)
#undef MOGT_CASE
    return set_error(MOGT_E_INVALID, "reverse diag scan: tile (vec=%d, lanes=%d, steps=%d, waves=%d) not compiled",
                     t.vec, t.lanes, t.steps, t.waves);
}

}  // namespace mogt
