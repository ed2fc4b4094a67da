// Coupled write-forget per-rank scan of the MOGT mixer (identity connection):
// the gate sigmoid, the coupling a = damping * (1 - g) and the gated write
// b = v * g are computed in registers inside the single-pass diagonal scan
// (diag_kernel.h), so the reference's [B, L, r, r] fp32 U, its [B, L, 3d] gate
// input and its gated V (model_mogt.py:104-182) are never written to memory.
#include "diag_kernel.h"

namespace mogt {

namespace {

template <typename TZ, typename TV, typename TO>
int coupled_dispatch(const DiagParams& prm, const DiagTile& t, hipStream_t st) {
#define MOGT_CASE(V_, F_, S_, W_)                                          \
    if (t.vec == V_ && t.lanes == F_ && t.steps == S_ && t.waves == W_) \
        return diag_launch<MODE_COUPLED, TV, TZ, TO, V_, F_, S_, W_, false>(prm, st);
    MOGT_COUPLED_TILES(MOGT_CASE)
#undef MOGT_CASE
    return set_error(MOGT_E_INVALID, "coupled scan: tile (vec=%d, lanes=%d, steps=%d, waves=%d) not compiled",
                     t.vec, t.lanes, t.steps, t.waves);
}

bool dtype_ok(int d) { return d == MOGT_F32 || d == MOGT_BF16; }

// Default tile (measured on MI355X at r = 16, c = 48, L = 8k..32k): four
// channels per lane where the channel count and the pointers allow it (the
// lanes of one vector must share a gate, so the vector must divide the channel
// count), 512-step chunks; short problems fall back to shorter chunks.
DiagTile coupled_tile(int64_t B, int64_t L, int64_t R, int64_t C, int align_elems) {
    static const TileChoice v4[] = {{{4, 16, 8, 16}, 512}, {{4, 16, 8, 8}, 128}, {{2, 32, 8, 16}, 128},
                                    {{1, 64, 8, 16}, 0}};
    static const TileChoice v2[] = {{{2, 32, 16, 8}, 128}, {{2, 32, 8, 16}, 128}, {{1, 64, 8, 16}, 0}};
    static const TileChoice v1[] = {{{1, 64, 32, 16}, 128}, {{1, 64, 16, 16}, 128}, {{1, 64, 8, 16}, 0}};
    if (C % 4 == 0 && align_elems % 4 == 0) return pick_tile(B, L, R * C, v4, 4);
    if (C % 2 == 0 && align_elems % 2 == 0) return pick_tile(B, L, R * C, v2, 3);
    return pick_tile(B, L, R * C, v1, 3);
}

// Largest vector width (4, 2 or 1 elements) both v and h are aligned to.
int coupled_alignment(const void* v, const void* h, int v_dtype, int out_dtype) {
    const uintptr_t ve = v_dtype == MOGT_BF16 ? 2 : 4, he = out_dtype == MOGT_BF16 ? 2 : 4;
    for (int n : {4, 2})
        if (reinterpret_cast<uintptr_t>(v) % (ve * n) == 0 && reinterpret_cast<uintptr_t>(h) % (he * n) == 0)
            return n;
    return 1;
}

}  // namespace

int coupled_run(const void* z, const void* v, void* h, int64_t B, int64_t L, int64_t R, int64_t C,
                float damping, int z_dtype, int v_dtype, int out_dtype, const DiagTile& t,
                void* ws, size_t ws_bytes, void* stream) {
    const int64_t D = R * C;
    if (C % t.vec != 0)
        return set_error(MOGT_E_INVALID, "channels %lld not a multiple of vec %d", (long long)C, t.vec);
    DiagParams prm{};
    int rc = diag_prepare(prm, B, L, D, t, ws, ws_bytes);
    if (rc) return rc;
    prm.a = z;
    prm.b = v;
    prm.h = h;
    prm.aprefix = nullptr;
    prm.R = static_cast<int>(R);
    prm.C = static_cast<int>(C);
    prm.damping = damping;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool zb = z_dtype == MOGT_BF16, vb = v_dtype == MOGT_BF16, ob = out_dtype == MOGT_BF16;
    if (!zb && vb && !ob) return coupled_dispatch<float, bf16_t, float>(prm, t, st);
    if (!zb && vb && ob) return coupled_dispatch<float, bf16_t, bf16_t>(prm, t, st);
    if (zb && vb && !ob) return coupled_dispatch<bf16_t, bf16_t, float>(prm, t, st);
    if (zb && vb && ob) return coupled_dispatch<bf16_t, bf16_t, bf16_t>(prm, t, st);
    if (!zb && !vb && !ob) return coupled_dispatch<float, float, float>(prm, t, st);
    if (!zb && !vb && ob) return coupled_dispatch<float, float, bf16_t>(prm, t, st);
    if (zb && !vb && !ob) return coupled_dispatch<bf16_t, float, float>(prm, t, st);
    return coupled_dispatch<bf16_t, float, bf16_t>(prm, t, st);
}

}  // namespace mogt

using namespace mogt;

extern "C" size_t mogt_coupled_rank_scan_workspace_bytes(int64_t batch, int64_t length,
                                                         int64_t rank, int64_t channels,
                                                         int v_dtype) {
    if (batch <= 0 || length <= 0 || rank <= 0 || channels <= 0) return WS_HDR_BYTES;
    // Largest requirement over the tiles the entry point may pick.
    (void)v_dtype;
    size_t best = 0;
    for (int al : {4, 2, 1}) {
        const size_t n = diag_geometry(batch, length, rank * channels,
                                       coupled_tile(batch, length, rank, channels, al)).bytes;
        best = n > best ? n : best;
    }
    return best;
}

extern "C" int mogt_coupled_rank_scan_fwd(const void* z, const void* v, void* h, int64_t batch,
                                          int64_t length, int64_t rank, int64_t channels,
                                          float damping, int z_dtype, int v_dtype, int out_dtype,
                                          void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    if (batch < 0 || length < 0) return set_error(MOGT_E_INVALID, "negative size");
    if (rank <= 0 || channels <= 0 || rank > 0x7fffffff || channels > 0x7fffffff)
        return set_error(MOGT_E_INVALID, "rank and channels must be positive");
    if (!dtype_ok(z_dtype) || !dtype_ok(v_dtype) || !dtype_ok(out_dtype))
        return set_error(MOGT_E_INVALID, "unsupported dtype code");
    if (batch == 0 || length == 0) return MOGT_OK;
    if (!z || !v || !h) return set_error(MOGT_E_INVALID, "null tensor pointer");
    const DiagTile t = coupled_tile(batch, length, rank, channels,
                                    coupled_alignment(v, h, v_dtype, out_dtype));
    return coupled_run(z, v, h, batch, length, rank, channels, damping, z_dtype, v_dtype, out_dtype,
                       t, workspace, workspace_bytes, stream);
}
