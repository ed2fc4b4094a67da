// Instantiations of the reverse-time diagonal scans (the backward recurrence
// G_t = dH_t + a_{t+1} G_{t+1}, see MODE_DIAG_REV / MODE_COUPLED_REV in
// diag_kernel.h): fp32 in, fp32 out, the tiles of the fp32 default lists.
#include "diag_kernel.h"

namespace mogt {

#define MOGT_DIAG_REV_TILES(X) X(2, 32, 32, 8) X(2, 32, 32, 4) X(2, 32, 16, 8) X(2, 32, 8, 16) X(1, 64, 32, 16) X(1, 64, 16, 16) X(1, 64, 8, 16)

int diag_run_rev(const DiagParams& prm, const DiagTile& t, hipStream_t st) {
#define MOGT_CASE(V_, F_, S_, W_)                                                         \
    if (t.vec == V_ && t.lanes == F_ && t.steps == S_ && t.waves == W_)                   \
        return diag_launch<MODE_DIAG_REV, float, float, float, V_, F_, S_, W_, false>(prm, st);
    MOGT_DIAG_REV_TILES(MOGT_CASE)
#undef MOGT_CASE
    return set_error(MOGT_E_INVALID, "reverse diag scan: tile (vec=%d, lanes=%d, steps=%d, waves=%d) not compiled",
                     t.vec, t.lanes, t.steps, t.waves);
}

namespace {

template <typename TZ>
int coupled_rev_dispatch(const DiagParams& prm, const DiagTile& t, hipStream_t st) {
#define MOGT_CASE(V_, F_, S_, W_)                                       \
    if (t.vec == V_ && t.lanes == F_ && t.steps == S_ && t.waves == W_) \
        return diag_launch<MODE_COUPLED_REV, float, TZ, float, V_, F_, S_, W_, false>(prm, st);
    MOGT_DIAG_REV_TILES(MOGT_CASE)
#undef MOGT_CASE
    return set_error(MOGT_E_INVALID, "coupled reverse scan: tile (vec=%d, lanes=%d, steps=%d, waves=%d) not compiled",
                     t.vec, t.lanes, t.steps, t.waves);
}

}  // namespace
}  // namespace mogt

using namespace mogt;

// Reverse scan of the coupled write-forget scan: G_t = dh_t + a_{t+1} G_{t+1}
// with a_t = damping * (1 - sigmoid(z[b, t, i])) over rank i's C channels,
// formed in registers from the gate logits (the [B, L, R*C] decay tensor of
// the generic reverse scan is never written).
extern "C" int mogt_coupled_rank_scan_rev_fwd(const void* z, const float* dh, float* G, int64_t batch,
                                              int64_t length, int64_t rank, int64_t channels, float damping,
                                              int z_dtype, void* workspace, size_t workspace_bytes,
                                              void* stream) {
    clear_error();
    if (batch < 0 || length < 0) return set_error(MOGT_E_INVALID, "negative size");
    if (rank <= 0 || channels <= 0 || rank > 0x7fffffff || channels > 0x7fffffff)
        return set_error(MOGT_E_INVALID, "rank and channels must be positive");
    if (z_dtype != MOGT_F32 && z_dtype != MOGT_BF16) return set_error(MOGT_E_INVALID, "unsupported dtype code");
    if (batch == 0 || length == 0) return MOGT_OK;
    if (!z || !dh || !G) return set_error(MOGT_E_INVALID, "null tensor pointer");
    const int64_t D = rank * channels;
    const bool vec2 = channels % 2 == 0 && reinterpret_cast<uintptr_t>(dh) % 8 == 0 &&
                      reinterpret_cast<uintptr_t>(G) % 8 == 0;
    // the fp32 default tile; two features per lane only where the lanes of a
    // vector share a gate (an even channel count) and the pointers allow
    const DiagTile t = f32_tile(batch, length, D, vec2);
    DiagParams prm{};
    const int rc = diag_prepare(prm, batch, length, D, t, workspace, workspace_bytes);
    if (rc) return rc;
    prm.a = z;
    prm.b = dh;
    prm.h = G;
    prm.aprefix = nullptr;
    prm.R = static_cast<int>(rank);
    prm.ldz = prm.R;
    prm.C = static_cast<int>(channels);
    prm.damping = damping;
    hipStream_t st = static_cast<hipStream_t>(stream);
    return z_dtype == MOGT_BF16 ? coupled_rev_dispatch<bf16_t>(prm, t, st)
                                : coupled_rev_dispatch<float>(prm, t, st);
}
