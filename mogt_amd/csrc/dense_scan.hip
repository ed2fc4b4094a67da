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

// The backward's reverse-time recurrence G_t = X_t + U_{t+1}^T G_{t+1}
// (affine_scan.py:110-118): level 0 in reversed time with U read transposed
// (the REV passes), the carries of its chunk summaries by the ordinary
// recursion (they are already in reversed order), then G once.
int run_rev(const float* U, const float* X, float* G, int64_t B, int64_t L, int64_t R, int64_t C, char* ws,
            const DenseGeo& geo, hipStream_t st) {
    ChunkParams c{};
    c.U = U; c.V = X;
    c.L = L; c.R = static_cast<int>(R); c.C = static_cast<int>(C); c.T = kDenseChunk;
    c.nb = static_cast<int>((L + c.T - 1) / c.T);
    c.withP = 0;
    c.outH = G;
    if (c.nb > 1) {
        const Level& v = geo.lv[0];
        ChunkParams s = c;
        s.sumP = reinterpret_cast<float*>(ws + v.sumP);
        s.sumH = reinterpret_cast<float*>(ws + v.sumH);
        int rc = dense_launch_pass<float, float, CM_SUMMARY, false, true>(s, B, st);
        if (rc) return rc;
        rc = excl_scan<float>(s.sumP, s.sumH, c.nb, reinterpret_cast<float*>(ws + v.carP),
                              reinterpret_cast<float*>(ws + v.carH), B, R, C, false, ws, geo, 1, st);
        if (rc) return rc;
        c.carH = reinterpret_cast<float*>(ws + v.carH);
    }
    return dense_launch_pass<float, float, CM_OUTPUT, false, true>(c, B, st);
}

// dU_t = G_t M_{t-1}^T for the augmented state M = [H | P] of the forward
// scan (P: the prefix products, only when their gradient is part of G), with
// M_{-1} = [0 | I]: the dU of affine_scan_sequential_backward
// (affine_scan.py:119-124) on the augmented state.  One work-group per step
// (b, t); G_t and M_{t-1} are staged through LDS 64 columns at a time (rows
// padded by one float: the 16 or 32 rows a wave reads at one column fall in
// distinct banks), and thread o accumulates elements o, o + 256, ... of the
// R x R output.
constexpr int kGuCols = 64;
__global__ __launch_bounds__(256) void dense_grad_u_kernel(const float* __restrict__ G, const float* __restrict__ H,
                                                           const float* __restrict__ P, float* __restrict__ dU,
                                                           int64_t L, int R, int C, int CG) {
    __shared__ float sG[32][kGuCols + 1];
    __shared__ float sM[32][kGuCols + 1];
    const int64_t row = blockIdx.x;            // b * L + t
    const int64_t t = row % L;
    const int tid = threadIdx.x;
    const int RR = R * R;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int c0 = 0; c0 < CG; c0 += kGuCols) {
        for (int e = tid; e < R * kGuCols; e += 256) {
            const int i = e / kGuCols, cc = e - i * kGuCols, c = c0 + cc;
            float gv = 0.0f, mv = 0.0f;
            if (c < CG) {
                gv = G[(row * R + i) * CG + c];
                if (c < C) mv = t > 0 ? H[((row - 1) * R + i) * C + c] : 0.0f;
                else mv = t > 0 ? P[((row - 1) * R + i) * R + (c - C)] : (i == c - C ? 1.0f : 0.0f);
            }
            sG[i][cc] = gv;
            sM[i][cc] = mv;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int o = tid + 256 * k;
            if (o < RR) {
                const int i = o / R, j = o - (o / R) * R;
                float a = acc[k];
#pragma unroll 8
                for (int cc = 0; cc < kGuCols; ++cc) a = fmaf(sG[i][cc], sM[j][cc], a);
                acc[k] = a;
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int o = tid + 256 * k;
        if (o < RR) dU[row * RR + o] = acc[k];
    }
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

extern "C" int mogt_affine_scan_rev_fwd(const void* U, const void* X, void* G, int64_t batch, int64_t length,
                                        int64_t rank, int64_t channels, void* workspace, size_t workspace_bytes,
                                        void* stream) {
    clear_error();
    int rc = check_dense_shapes(batch, length, rank, channels);
    if (rc) return rc;
    if (channels == 0) return set_error(MOGT_E_INVALID, "the reverse scan needs C > 0");
    if (batch == 0 || length == 0) return MOGT_OK;
    if (!U || !X || !G) return set_error(MOGT_E_INVALID, "null tensor pointer");
    if (batch > 65535 || (length + kDenseChunk - 1) / kDenseChunk > 0x7fffffffLL)
        return set_error(MOGT_E_INVALID, "problem too large for one launch");
    const DenseGeo g = dense_geometry(batch, length, rank, channels);
    if (!workspace || workspace_bytes < g.bytes)
        return set_error(MOGT_E_WORKSPACE, "workspace of %zu bytes required, got %zu", g.bytes, workspace_bytes);
    return run_rev(static_cast<const float*>(U), static_cast<const float*>(X), static_cast<float*>(G), batch, length,
                   rank, channels, static_cast<char*>(workspace), g, static_cast<hipStream_t>(stream));
}

extern "C" int mogt_affine_scan_grad_u(const void* G, const void* H, const void* P, void* dU, int64_t batch,
                                       int64_t length, int64_t rank, int64_t channels, void* stream) {
    clear_error();
    if (batch < 0 || length < 0 || rank <= 0 || channels < 0)
        return set_error(MOGT_E_INVALID, "G must be [B, L, R, C (+ R)], H [B, L, R, C]");
    if (rank > 32) return set_error(MOGT_E_INVALID, "R = %lld not supported (R <= 32)", (long long)rank);
    if (channels > (1 << 22)) return set_error(MOGT_E_INVALID, "C too large");
    if (batch == 0 || length == 0) return MOGT_OK;
    if (!G || !dU || (channels > 0 && !H) || (channels == 0 && !P))
        return set_error(MOGT_E_INVALID, "null tensor pointer");
    if (batch * length > 0x7fffffffLL) return set_error(MOGT_E_INVALID, "problem too large for one launch");
    const int CG = static_cast<int>(channels + (P ? rank : 0));
    hipLaunchKernelGGL(dense_grad_u_kernel, dim3(static_cast<unsigned>(batch * length)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const float*>(G),
                       static_cast<const float*>(H), static_cast<const float*>(P), static_cast<float*>(dU),
                       length, static_cast<int>(rank), static_cast<int>(channels), CG);
    return check_launch("dense_grad_u_kernel");
}
