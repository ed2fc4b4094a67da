// Dense affine scan H_t = U_t H_{t-1} + V_t (U_t: R x R, H/V: R x C) for gfx950:
// host recursion and C-ABI entry points.  The chunk kernel and its launch
// dispatch live in dense_kernel.h (instantiated by dense_pass_*.hip).
//
// Semantics: affine_scan_sequential (affine_scan.py:14-62), fp32 state, H_0 = 0,
// optional prefix products P_t = U_t ... U_1; the chunk/carry decomposition of
// affine_scan_block_reference (affine_scan.py:175-278) and the reference's
// hybrid path (triton_scan.py:232-311).
//
// The carries are themselves an affine scan: (P_T, H_T) of consecutive chunks
// compose exactly like (U_t, V_t) -- the reference's affine_combine
// (affine_scan.py:4-11), (P_a, H_a) o (P_b, H_b) = (P_a P_b, P_a H_b + H_a).
// So the chunk summaries, laid out like U and V, are scanned by the same
// kernel, recursively: summaries of summaries until one chunk remains, then
// EXCL passes back down produce every level's carries, and the OUTPUT pass of
// level 0 writes H once.  Each pass is independent per chunk (no inter-chunk
// waits).  With 32-step chunks, L = 32768 needs five passes (1024 -> 32 -> 1).
#include "dense_kernel.h"

namespace mogt {
namespace {

// Workspace: per level l >= 0 with n_l = ceil(n_{l-1} / T) chunks (n_{-1} = L),
// the chunk products (sumP, sumH) and the chunk carries (carP, carH), fp32.
struct Level {
    int64_t n;                        // chunks of this level (= steps of the next)
    size_t sumP, sumH, carP, carH;    // byte offsets
};
struct DenseGeo {
    int depth;
    Level lv[24];
    size_t bytes;
};

DenseGeo dense_geometry(int64_t B, int64_t L, int64_t R, int64_t C) {
    DenseGeo g{};
    size_t off = WS_HDR_BYTES;
    auto take = [&](size_t nbytes) { size_t o = off; off = round_up(off + nbytes, 256); return o; };
    int64_t steps = L;
    while (steps > 1 && g.depth < 24) {
        const int T = kDenseChunk;
        Level& v = g.lv[g.depth++];
        v.n = (steps + T - 1) / T;
        const size_t m = static_cast<size_t>(B) * v.n;
        v.sumP = take(m * R * R * sizeof(float));
        v.sumH = take(m * R * static_cast<size_t>(C) * sizeof(float));
        v.carP = take(m * R * R * sizeof(float));
        v.carH = take(m * R * static_cast<size_t>(C) * sizeof(float));
        steps = v.n;
    }
    g.bytes = off;
    return g;
}

// Exclusive scan of a level's (U, V) sequence of `len` steps into (outP, outH):
// the state before every step, starting from [I | 0].  Recursive over chunk
// products; lv indexes the workspace level holding this sequence's chunks.
template <typename TV>
int excl_scan(const float* U, const void* V, int64_t len, float* outP, float* outH, int64_t B,
              int64_t R, int64_t C, bool withP, char* ws, const DenseGeo& geo, int lv,
              hipStream_t st) {
    ChunkParams c{};
    c.U = U; c.V = C > 0 ? V : nullptr;
    c.L = len; c.R = static_cast<int>(R); c.C = static_cast<int>(C); c.T = kDenseChunk;
    c.nb = static_cast<int>((len + c.T - 1) / c.T);
    c.withP = withP;
    c.outP = withP ? outP : nullptr;
    c.outH = outH;
    if (c.nb > 1) {
        const Level& v = geo.lv[lv];
        ChunkParams s = c;
        s.sumP = reinterpret_cast<float*>(ws + v.sumP);
        s.sumH = reinterpret_cast<float*>(ws + v.sumH);
        int rc = dense_launch_pass<TV, float, CM_SUMMARY>(s, B, st);
        if (rc) return rc;
        // carries of this level's chunks: exclusive scan of the chunk products
        rc = excl_scan<float>(s.sumP, s.sumH, c.nb, reinterpret_cast<float*>(ws + v.carP),
                              reinterpret_cast<float*>(ws + v.carH), B, R, C, withP, ws, geo, lv + 1, st);
        if (rc) return rc;
        c.carP = withP ? reinterpret_cast<float*>(ws + v.carP) : nullptr;
        c.carH = reinterpret_cast<float*>(ws + v.carH);
    }
    return dense_launch_pass<TV, float, CM_EXCL>(c, B, st);
}

// Level 0 (VK: V_t = v_t k_t^T from V = v, K = k), then the carries, then H.
template <typename TV, typename TO, bool VK>
int run_levels(const float* U, const void* V, const void* K, void* H, void* P, int64_t B, int64_t L,
               int64_t R, int64_t C, char* ws, const DenseGeo& geo, hipStream_t st) {
    const bool withP = P != nullptr;
    ChunkParams c{};
    c.U = U; c.V = C > 0 ? V : nullptr; c.K = VK ? K : nullptr;
    c.L = L; c.R = static_cast<int>(R); c.C = static_cast<int>(C); c.T = kDenseChunk;
    c.nb = static_cast<int>((L + c.T - 1) / c.T);
    c.withP = withP;
    c.outP = P; c.outH = H;
    if (c.nb > 1) {
        const Level& v = geo.lv[0];
        ChunkParams s = c;
        s.sumP = reinterpret_cast<float*>(ws + v.sumP);
        s.sumH = reinterpret_cast<float*>(ws + v.sumH);
        int rc = dense_launch_pass<TV, float, CM_SUMMARY, VK>(s, B, st);
        if (rc) return rc;
        rc = excl_scan<float>(s.sumP, s.sumH, c.nb, reinterpret_cast<float*>(ws + v.carP),
                              reinterpret_cast<float*>(ws + v.carH), B, R, C, withP, ws, geo, 1, st);
        if (rc) return rc;
        c.carP = withP ? reinterpret_cast<float*>(ws + v.carP) : nullptr;
        c.carH = reinterpret_cast<float*>(ws + v.carH);
    }
    return dense_launch_pass<TV, TO, CM_OUTPUT, VK>(c, B, st);
}

int check_dense_shapes(int64_t B, int64_t L, int64_t R, int64_t C) {
    if (B < 0 || L < 0 || R <= 0 || C < 0)
        return set_error(MOGT_E_INVALID, "U must be [B, L, R, R] and V must be [B, L, R, C]");
    if (R > 32) return set_error(MOGT_E_INVALID, "R = %lld not supported (R <= 32)", (long long)R);
    if (C > (1 << 22)) return set_error(MOGT_E_INVALID, "C too large");
    return MOGT_OK;
}

// K != nullptr: the rank-1 form, V holds v [B, L, R] and K holds k [B, L, C].
int run_dense(const float* U, const void* V, const void* K, void* H, void* P, int64_t B, int64_t L,
              int64_t R, int64_t C, int v_dtype, int out_dtype, void* ws, size_t ws_bytes, void* stream) {
    clear_error();
    int rc = check_dense_shapes(B, L, R, C);
    if (rc) return rc;
    if (v_dtype != MOGT_F32 && v_dtype != MOGT_BF16) return set_error(MOGT_E_INVALID, "unsupported V dtype");
    if (out_dtype != MOGT_F32 && out_dtype != MOGT_BF16) return set_error(MOGT_E_INVALID, "unsupported output dtype");
    if (B == 0 || L == 0) return MOGT_OK;
    if (!U || (C > 0 && (!V || !H)) || (C == 0 && !P)) return set_error(MOGT_E_INVALID, "null tensor pointer");
    if (B > 65535 || (L + kDenseChunk - 1) / kDenseChunk > 0x7fffffffLL)
        return set_error(MOGT_E_INVALID, "problem too large for one launch");
    const DenseGeo g = dense_geometry(B, L, R, C);
    if (!ws || ws_bytes < g.bytes)
        return set_error(MOGT_E_WORKSPACE, "workspace of %zu bytes required, got %zu", g.bytes, ws_bytes);
    char* base = static_cast<char*>(ws);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool vf = v_dtype == MOGT_F32, of = out_dtype == MOGT_F32;
    if (K) {
        if (vf && of) return run_levels<float, float, true>(U, V, K, H, P, B, L, R, C, base, g, st);
        if (vf) return run_levels<float, bf16_t, true>(U, V, K, H, P, B, L, R, C, base, g, st);
        if (of) return run_levels<bf16_t, float, true>(U, V, K, H, P, B, L, R, C, base, g, st);
        return run_levels<bf16_t, bf16_t, true>(U, V, K, H, P, B, L, R, C, base, g, st);
    }
    if (vf && of) return run_levels<float, float, false>(U, V, K, H, P, B, L, R, C, base, g, st);
    if (vf) return run_levels<float, bf16_t, false>(U, V, K, H, P, B, L, R, C, base, g, st);
    if (of) return run_levels<bf16_t, float, false>(U, V, K, H, P, B, L, R, C, base, g, st);
    return run_levels<bf16_t, bf16_t, false>(U, V, K, H, P, B, L, R, C, base, g, st);
}

}  // namespace
}  // namespace mogt

using namespace mogt;

extern "C" size_t mogt_affine_scan_workspace_bytes(int64_t batch, int64_t length, int64_t rank,
                                                   int64_t channels) {
    if (batch <= 0 || length <= 0 || rank <= 0 || rank > 32 || channels < 0) return WS_HDR_BYTES;
    return dense_geometry(batch, length, rank, channels).bytes;
}

extern "C" int mogt_affine_scan_fwd(const void* U, const void* V, void* H, void* U_prefix, int64_t batch,
                                    int64_t length, int64_t rank, int64_t channels, int v_dtype,
                                    int out_dtype, void* workspace, size_t workspace_bytes,
                                    void* stream) {
    return run_dense(static_cast<const float*>(U), V, nullptr, H, U_prefix, batch, length, rank, channels,
                     v_dtype, out_dtype, workspace, workspace_bytes, stream);
}

extern "C" int mogt_affine_scan_vk_fwd(const void* U, const void* v, const void* k, void* H, void* U_prefix,
                                       int64_t batch, int64_t length, int64_t rank, int64_t channels,
                                       int vk_dtype, int out_dtype, void* workspace, size_t workspace_bytes,
                                       void* stream) {
    // empty problems return before any pointer is needed (as in run_dense)
    if (batch > 0 && length > 0 && channels > 0 && (!v || !k)) {
        clear_error();
        return set_error(MOGT_E_INVALID, "null tensor pointer");
    }
    return run_dense(static_cast<const float*>(U), v, channels > 0 ? k : nullptr, H, U_prefix, batch, length,
                     rank, channels, vk_dtype, out_dtype, workspace, workspace_bytes, stream);
}

extern "C" size_t mogt_fused_scan_workspace_bytes(int64_t batch, int64_t length, int64_t rank) {
    return mogt_affine_scan_workspace_bytes(batch, length, rank, 0);
}

extern "C" int mogt_fused_scan_fwd(const void* U, void* Y, int64_t batch, int64_t length, int64_t rank,
                                   int out_dtype, void* workspace, size_t workspace_bytes,
                                   void* stream) {
    return run_dense(static_cast<const float*>(U), nullptr, nullptr, nullptr, Y, batch, length, rank, 0,
                     MOGT_F32, out_dtype, workspace, workspace_bytes, stream);
}

extern "C" int mogt_affine_local_scan(const void* U, const void* V, void* U_prefix, void* H_prefix,
                                      void* U_summary, void* H_summary, int64_t batch, int64_t length,
                                      int64_t rank, int64_t channels, int64_t block_size, int v_dtype,
                                      void* stream) {
    clear_error();
    int rc = check_dense_shapes(batch, length, rank, channels);
    if (rc) return rc;
    if (block_size <= 0) return set_error(MOGT_E_INVALID, "block_size must be positive");
    if (v_dtype != MOGT_F32 && v_dtype != MOGT_BF16) return set_error(MOGT_E_INVALID, "unsupported V dtype");
    if (batch == 0 || length == 0) return MOGT_OK;
    if (!U || !U_prefix || !U_summary || (channels > 0 && (!V || !H_prefix || !H_summary)))
        return set_error(MOGT_E_INVALID, "null tensor pointer");
    const int64_t nb = (length + block_size - 1) / block_size;
    if (nb > 0x7fffffffLL || block_size > 0x7fffffffLL || batch > 65535)
        return set_error(MOGT_E_INVALID, "problem too large for one launch");
    ChunkParams c{};
    c.U = static_cast<const float*>(U);
    c.V = channels > 0 ? V : nullptr;
    c.outP = U_prefix; c.outH = H_prefix;
    c.sumP = static_cast<float*>(U_summary);
    c.sumH = static_cast<float*>(H_summary);
    c.L = length; c.R = static_cast<int>(rank); c.C = static_cast<int>(channels);
    c.T = static_cast<int>(block_size); c.nb = static_cast<int>(nb);
    c.withP = 1;
    hipStream_t st = static_cast<hipStream_t>(stream);
    return v_dtype == MOGT_BF16 ? dense_launch_pass<bf16_t, float, CM_LOCAL>(c, batch, st)
                                : dense_launch_pass<float, float, CM_LOCAL>(c, batch, st);
}
