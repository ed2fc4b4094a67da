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
    MOGT_COUPLED_REV_TILES(MOGT_CASE)
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
namespace {

int coupled_rev_run(const void* z, const float* dh, float* G, int64_t batch, int64_t length, int64_t rank,
                    int64_t channels, float damping, int z_dtype, const DiagTile& t, void* workspace,
                    size_t workspace_bytes, void* stream) {
    const int64_t D = rank * channels;
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

int coupled_rev_check(const void* z, const float* dh, float* G, int64_t batch, int64_t length, int64_t rank,
                      int64_t channels, int z_dtype) {
    if (batch < 0 || length < 0) return set_error(MOGT_E_INVALID, "negative size");
    if (rank <= 0 || channels <= 0 || rank > 0x7fffffff || channels > 0x7fffffff)
        return set_error(MOGT_E_INVALID, "rank and channels must be positive");
    if (z_dtype != MOGT_F32 && z_dtype != MOGT_BF16) return set_error(MOGT_E_INVALID, "unsupported dtype code");
    if (batch == 0 || length == 0) return MOGT_OK;
    if (!z || !dh || !G) return set_error(MOGT_E_INVALID, "null tensor pointer");
    return 1;
}

}  // namespace

namespace {

// Default tile (measured on MI355X at r = 16, c = 48, L = 8K..32K): four
// channels per lane, 8 steps, 8 waves (78 VGPRs: three work-groups per CU, so
// L = 32768's 1536 chunks of 256 steps run as two full generations; the fp32
// diagonal tile (2, 32, 32, 8) needs 173 VGPRs, one work-group per CU): 48.2
// -> 44.5 us at L = 32768.  Elsewhere the fp32 default tile, two features per
// lane only where the lanes of a vector share a gate (an even channel count)
// and the pointers allow.  `align` is the largest vector (4, 2, 1 fp32
// elements) dh and G are aligned to.
DiagTile coupled_rev_tile(int64_t B, int64_t L, int64_t R, int64_t C, int align) {
    if (C % 4 == 0 && align % 4 == 0) return DiagTile{4, 16, 8, 8};
    return f32_tile(B, L, R * C, C % 2 == 0 && align % 2 == 0);
}

}  // namespace

extern "C" size_t mogt_coupled_rank_scan_rev_workspace_bytes(int64_t batch, int64_t length, int64_t rank,
                                                             int64_t channels) {
    if (batch <= 0 || length <= 0 || rank <= 0 || channels <= 0) return WS_HDR_BYTES;
    size_t best = 0;
    for (int al : {4, 2, 1}) {
        const size_t n = diag_geometry(batch, length, rank * channels,
                                       coupled_rev_tile(batch, length, rank, channels, al)).bytes;
        best = n > best ? n : best;
    }
    return best;
}

extern "C" int mogt_coupled_rank_scan_rev_fwd(const void* z, const float* dh, float* G, int64_t batch,
                                              int64_t length, int64_t rank, int64_t channels, float damping,
                                              int z_dtype, void* workspace, size_t workspace_bytes,
                                              void* stream) {
    clear_error();
    const int ok = coupled_rev_check(z, dh, G, batch, length, rank, channels, z_dtype);
    if (ok <= 0) return ok;
    const uintptr_t pa = reinterpret_cast<uintptr_t>(dh) | reinterpret_cast<uintptr_t>(G);
    const int align = pa % 16 == 0 ? 4 : (pa % 8 == 0 ? 2 : 1);
    const DiagTile t = coupled_rev_tile(batch, length, rank, channels, align);
    return coupled_rev_run(z, dh, G, batch, length, rank, channels, damping, z_dtype, t, workspace, workspace_bytes,
                           stream);
}

// The same with an explicit tile, one of mogt_diag_scan_tiles(3) whose vector
// divides the channel count (dh and G aligned to it, up to 16 bytes).
extern "C" int mogt_coupled_rank_scan_rev_fwd_cfg(const void* z, const float* dh, float* G, int64_t batch,
                                                  int64_t length, int64_t rank, int64_t channels, float damping,
                                                  int z_dtype, int vec, int lanes, int steps, int waves,
                                                  void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    const DiagTile t{vec, lanes, steps, waves};
    if (!diag_tile_compiled(3, t))
        return set_error(MOGT_E_INVALID, "coupled reverse scan: tile (%d,%d,%d,%d) not compiled", vec, lanes, steps,
                         waves);
    const int ok = coupled_rev_check(z, dh, G, batch, length, rank, channels, z_dtype);
    if (ok <= 0) return ok;
    if (channels % vec != 0)
        return set_error(MOGT_E_INVALID, "channels %lld not a multiple of vec %d", (long long)channels, vec);
    const uintptr_t bytes = static_cast<uintptr_t>(vec) * 4;
    if (reinterpret_cast<uintptr_t>(dh) % bytes || reinterpret_cast<uintptr_t>(G) % bytes)
        return set_error(MOGT_E_INVALID, "dh and G must be aligned to the tile's vector");
    return coupled_rev_run(z, dh, G, batch, length, rank, channels, damping, z_dtype, t, workspace, workspace_bytes,
                           stream);
}
